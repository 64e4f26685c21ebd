// DecoderTransformerGpu / KvCacheGpu: the caller of the GEMM + attention hot
// path, at M = B·T rows, plus its C ABI (aur_model_*, aur_kv_cache_*).
//
// Reference: src/gpu/transformer.rs (encode_forward :1347, train step
// :1535-1716, block_backward :1825-2005, AdamW :2008, prefill / decode
// :2374-2640) and the CPU model it must agree with, src/transformer/
// {model,block,attention,ffn,embedding,kv_cache}.rs.
//
// One step enqueues, per layer, 4 forward GEMMs (fused QKV, W_o with the
// residual add in its epilogue, fc with GELU in its epilogue, proj with the
// residual add), 4 dX GEMMs (GELU' fused into the proj-dX epilogue) and
// 4 weight-gradient accumulates, plus the flash attention forward / 3-pass
// backward and the row kernels of step_ops.hip.  Everything stays on the
// device; the host reads back only the per-row NLL (one small copy per step).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <vector>

#include "aurora.hpp"
#include "common.hpp"
#include "step_ops.hpp"

namespace aurora {

namespace {

constexpr float kLnEps = 1e-5f;  // LayerNorm::new (src/attention.rs:44)

// Bump allocator over one device allocation (256-byte aligned slices).
struct Carver {
  char* base;
  size_t off = 0;
  template <class T>
  T* take(size_t n) {
    off = (off + 255) & ~size_t(255);
    T* p = reinterpret_cast<T*>(base + off);
    off += n * sizeof(T);
    return p;
  }
};

inline void ck(aur_ctx* ctx, int rc, const char* what) { check(ctx, rc, what); }
inline void hip_ck(aur_ctx* ctx, hipError_t e, const char* what) {
  if (e != hipSuccess) check(ctx, aur::set_error(ctx, (int)e, "%s: %s", what, hipGetErrorString(e)), what);
}

// The largest split count <= s whose K ranges (multiples of 64, as
// gemm_nt_partials cuts them) are all non-empty.
int fit_splits(size_t K, int s) {
  for (s = std::max(s, 1); s > 1; --s) {
    const size_t chunk = ((K + s - 1) / s + 63) / 64 * 64;
    if ((K + chunk - 1) / chunk == (size_t)s) break;
  }
  return s;
}

// K ranges of the decode QKV projection (K = d_model): ranges of 128, at most
// 8 (the attention kernel sums at most 8).
int qkv_splits(size_t d) { return fit_splits(d, (int)std::max<size_t>(1, std::min<size_t>(8, d / 128))); }

// AUR_DEC_SPLITS = "q:o:p" overrides the decode step's split counts (QKV,
// W_o, W_proj; 0 keeps the default) for tuning; read when a cache is
// created.
int split_override(int which, int dflt, size_t K, int cap) {
  const char* env = std::getenv("AUR_DEC_SPLITS");
  if (!env) return dflt;
  int v[3] = {0, 0, 0};
  if (std::sscanf(env, "%d:%d:%d", &v[0], &v[1], &v[2]) < 1 || v[which] <= 0) return dflt;
  return fit_splits(K, std::min(v[which], cap));
}

}  // namespace

struct DecoderTransformerGpu::Layer {
  // parameters (views into the flat parameter buffer) and their gradients
  float *ln1_g, *ln1_b, *w_qkv, *w_o, *ln2_g, *ln2_b, *w_fc, *w_proj;
  float *g_ln1_g, *g_ln1_b, *g_w_qkv, *g_w_o, *g_ln2_g, *g_ln2_b, *g_w_fc, *g_w_proj;
  // saved activations of the last forward
  float *ln1, *mean1, *rstd1, *qkv, *attn, *lse, *xmid, *ln2, *mean2, *rstd2, *hpre, *hpost;
};

struct DecoderTransformerGpu::Acts {
  size_t rows;
  std::vector<float*> xs;  // residual stream: xs[l] = input of layer l, xs[L] = final
  float *lnf, *meanf, *rstdf, *logits, *nll;
  float *dx_a, *dx_b, *dln, *dh, *dqkv, *dattn;
  float *ln_ws, *attn_ws, *norm_part, *stats, *last;
  uint32_t *tok, *tgt, *csr_tok;
  int32_t *csr_off, *csr_idx;
  float *w_tok, *w_pos, *lnf_g, *lnf_b, *g_w_tok, *g_w_pos, *g_lnf_g, *g_lnf_b;
  std::vector<float> nll_host;
  // Pinned host staging of a training step's uploads (token ids, targets and
  // the embedding-gradient scatter plan), so they are copied asynchronously
  // and the plan is built on the host while the GPU runs the forward.
  // pin_done: recorded after the last copy out of it.
  uint32_t *pin = nullptr, *pin_tok = nullptr, *pin_tgt = nullptr, *pin_csr_tok = nullptr;
  int32_t *pin_csr_off = nullptr, *pin_csr_idx = nullptr;
  hipEvent_t pin_done = nullptr;
};

DecoderTransformerGpu::DecoderTransformerGpu(aur_ctx* ctx, const TransformerConfig& cfg,
                                             uint32_t max_batch)
    : ctx_(ctx), cfg_(cfg), max_batch_(max_batch) {
  // A constructor that throws runs no destructor: free what was allocated
  // before the failure (an activation arena too large for the device, say).
  try {
    init();
  } catch (...) {
    release();
    throw;
  }
}

void DecoderTransformerGpu::init() {
  const TransformerConfig& cfg = cfg_;
  aur_ctx* ctx = ctx_;
  const uint32_t max_batch = max_batch_;
  const size_t V = cfg.vocab, d = cfg.d_model, L = cfg.n_layer, F = cfg.d_ff, Tm = cfg.seq_len_max;
  if (!ctx || V == 0 || d == 0 || L == 0 || F == 0 || Tm == 0 || max_batch == 0 || cfg.n_head == 0 ||
      d % cfg.n_head != 0)
    throw Error("DecoderTransformerGpu: invalid config", AUR_EINVAL);
  // d_head up to 64, as the reference's one-thread-per-column attention
  // backward takes (src/gpu/attention.rs:266-331); multiples of 8 run the
  // attention kernels in place, any other d_head on zero-padded head copies
  // (training) and the generic KV kernel (decode).
  const uint32_t dh = cfg.d_model / cfg.n_head;
  if (dh > 64) throw Error("DecoderTransformerGpu: d_head must be at most 64", AUR_ELIMIT);
  if (d % 4 != 0 || F % 4 != 0 || V % 4 != 0)
    throw Error("DecoderTransformerGpu: vocab, d_model, d_ff must be multiples of 4", AUR_EINVAL);
  // Flat parameter layout: weight-decayed tensors first (w_tok, then per
  // layer w_qkv = [w_q; w_k; w_v], w_o, w_fc, w_proj), then the undecayed
  // ones (w_pos, per layer ln1_g, ln1_b, ln2_g, ln2_b, then lnf_g, lnf_b).
  n_decay_ = V * d + L * (3 * d * d + d * d + F * d + d * F);
  n_params_ = n_decay_ + Tm * d + L * 4 * d + 2 * d;
  // params | grads | m1 | m2 | Muon momentum (one float per matrix
  // parameter, [V·d, n_decay) of the flat layout).  The momentum exists from
  // the start, as the reference's GpuParams mu buffers do, so the persistent
  // state (and state_bytes()) has one fixed size.
  const size_t n_mu = n_decay_ - V * d;
  const size_t state_floats = 4 * n_params_ + n_mu;
  ck(ctx_, aur_malloc(ctx_, state_floats * sizeof(float) + 4096, &state_mem_), "alloc params");
  params_ = static_cast<float*>(state_mem_);
  grads_ = params_ + n_params_;
  m1_ = grads_ + n_params_;
  m2_ = m1_ + n_params_;
  mu_ = m2_ + n_params_;
  ck(ctx_, aur_memset0(ctx_, state_mem_, state_floats * sizeof(float)), "zero state");

  layers_ = new std::vector<Layer>(L);
  acts_ = new Acts();
  auto& A = *acts_;
  size_t off = 0;
  auto pv = [&](size_t n) {
    size_t o = off;
    off += n;
    return o;
  };
  const size_t o_wtok = pv(V * d);
  std::vector<size_t> o_qkv(L), o_wo(L), o_fc(L), o_proj(L);
  for (size_t l = 0; l < L; ++l) {
    o_qkv[l] = pv(3 * d * d);
    o_wo[l] = pv(d * d);
    o_fc[l] = pv(F * d);
    o_proj[l] = pv(d * F);
  }
  const size_t o_wpos = pv(Tm * d);
  std::vector<size_t> o_ln(L);
  for (size_t l = 0; l < L; ++l) o_ln[l] = pv(4 * d);
  const size_t o_lnf = pv(2 * d);
  A.w_tok = params_ + o_wtok;
  A.g_w_tok = grads_ + o_wtok;
  A.w_pos = params_ + o_wpos;
  A.g_w_pos = grads_ + o_wpos;
  A.lnf_g = params_ + o_lnf;
  A.lnf_b = A.lnf_g + d;
  A.g_lnf_g = grads_ + o_lnf;
  A.g_lnf_b = A.g_lnf_g + d;
  for (size_t l = 0; l < L; ++l) {
    Layer& Y = (*layers_)[l];
    Y.w_qkv = params_ + o_qkv[l];
    Y.w_o = params_ + o_wo[l];
    Y.w_fc = params_ + o_fc[l];
    Y.w_proj = params_ + o_proj[l];
    Y.ln1_g = params_ + o_ln[l];
    Y.ln1_b = Y.ln1_g + d;
    Y.ln2_g = Y.ln1_g + 2 * d;
    Y.ln2_b = Y.ln1_g + 3 * d;
    Y.g_w_qkv = grads_ + o_qkv[l];
    Y.g_w_o = grads_ + o_wo[l];
    Y.g_w_fc = grads_ + o_fc[l];
    Y.g_w_proj = grads_ + o_proj[l];
    Y.g_ln1_g = grads_ + o_ln[l];
    Y.g_ln1_b = Y.g_ln1_g + d;
    Y.g_ln2_g = Y.g_ln1_g + 2 * d;
    Y.g_ln2_b = Y.g_ln1_g + 3 * d;
  }

  // Activation arena for max_batch × seq_len_max rows.
  const size_t M = (size_t)max_batch * Tm;
  const size_t H = cfg.n_head;
  A.rows = M;
  const size_t per_layer = M * d /*ln1*/ + 2 * M /*stats*/ + 3 * M * d /*qkv*/ + M * d /*attn*/ +
                           H * M /*lse*/ + M * d /*xmid*/ + M * d /*ln2*/ + 2 * M + 2 * M * F;
  const size_t lnws = aur::layer_norm_backward_ws_floats((int)M, (int)d);
  // attention backward: rowdot + the causal dS tiles of max_batch sequences
  const size_t attn_ws_floats = aur::mha_bwd_tiled_ws_floats((int)max_batch, (int)Tm, (int)H);
  const size_t floats = L * per_layer + (L + 1) * M * d + M * d + 2 * M + M * V + M +
                        4 * M * d + M * F + 3 * M * d + lnws + attn_ws_floats + aur::grad_norm_ws_floats() + 16 +
                        (size_t)max_batch * d;
  const size_t ints = 3 * M + 2 * M + 2;
  const size_t bytes = floats * 4 + ints * 4 + 64 * 256 + 4096 * (L + 8);
  ck(ctx_, aur_malloc(ctx_, bytes, &act_mem_), "alloc activations");
  Carver cv{static_cast<char*>(act_mem_)};
  A.xs.resize(L + 1);
  for (size_t l = 0; l <= L; ++l) A.xs[l] = cv.take<float>(M * d);
  for (size_t l = 0; l < L; ++l) {
    Layer& Y = (*layers_)[l];
    Y.ln1 = cv.take<float>(M * d);
    Y.mean1 = cv.take<float>(M);
    Y.rstd1 = cv.take<float>(M);
    Y.qkv = cv.take<float>(3 * M * d);
    Y.attn = cv.take<float>(M * d);
    Y.lse = cv.take<float>(H * M);
    Y.xmid = cv.take<float>(M * d);
    Y.ln2 = cv.take<float>(M * d);
    Y.mean2 = cv.take<float>(M);
    Y.rstd2 = cv.take<float>(M);
    Y.hpre = cv.take<float>(M * F);
    Y.hpost = cv.take<float>(M * F);
  }
  A.lnf = cv.take<float>(M * d);
  A.meanf = cv.take<float>(M);
  A.rstdf = cv.take<float>(M);
  A.logits = cv.take<float>(M * V);
  A.nll = cv.take<float>(M);
  A.dx_a = cv.take<float>(M * d);
  A.dx_b = cv.take<float>(M * d);
  A.dln = cv.take<float>(M * d);
  A.dattn = cv.take<float>(M * d);
  A.dh = cv.take<float>(M * F);
  A.dqkv = cv.take<float>(3 * M * d);
  A.ln_ws = cv.take<float>(lnws);
  A.attn_ws = cv.take<float>(attn_ws_floats);
  A.norm_part = cv.take<float>(aur::grad_norm_ws_floats());
  A.stats = cv.take<float>(16);
  A.last = cv.take<float>((size_t)max_batch * d);
  A.tok = cv.take<uint32_t>(M);
  A.tgt = cv.take<uint32_t>(M);
  A.csr_tok = cv.take<uint32_t>(M);
  A.csr_off = cv.take<int32_t>(M + 1);
  A.csr_idx = cv.take<int32_t>(M);
  if (cv.off > bytes) throw Error("DecoderTransformerGpu: arena overflow", AUR_ENOMEM);
  if (hipHostMalloc(reinterpret_cast<void**>(&A.pin), (5 * M + 1) * sizeof(uint32_t)) != hipSuccess)
    throw Error("DecoderTransformerGpu: pinned staging allocation failed", AUR_ENOMEM);
  A.pin_tok = A.pin;
  A.pin_tgt = A.pin + M;
  A.pin_csr_tok = A.pin + 2 * M;
  A.pin_csr_idx = reinterpret_cast<int32_t*>(A.pin + 3 * M);
  A.pin_csr_off = reinterpret_cast<int32_t*>(A.pin + 4 * M);
  if (hipEventCreateWithFlags(&A.pin_done, hipEventDisableTiming) != hipSuccess)
    throw Error("DecoderTransformerGpu: event creation failed", AUR_ENOMEM);
}

DecoderTransformerGpu::~DecoderTransformerGpu() {
  for (KvCacheGpu* c : caches_) {
    c->drop_graph();
    c->owner_ = nullptr;
  }
  release();
}

void DecoderTransformerGpu::release() noexcept {
  if (ctx_) {
    aur_sync(ctx_);
    if (acts_ && acts_->pin) (void)hipHostFree(acts_->pin);
    if (acts_ && acts_->pin_done) (void)hipEventDestroy(acts_->pin_done);
    if (act_mem_) aur_free(ctx_, act_mem_);
    if (state_mem_) aur_free(ctx_, state_mem_);
    if (muon_mem_) aur_free(ctx_, muon_mem_);
  }
  act_mem_ = state_mem_ = muon_mem_ = nullptr;
  delete layers_;
  delete acts_;
  layers_ = nullptr;
  acts_ = nullptr;
}

float* DecoderTransformerGpu::tensor(const std::string& name, int layer, bool grad, size_t* n) const {
  const size_t V = cfg_.vocab, d = cfg_.d_model, F = cfg_.d_ff, Tm = cfg_.seq_len_max;
  const auto& A = *acts_;
  auto ret = [&](float* p, size_t len) {
    if (n) *n = len;
    return p;
  };
  if (name == "params") return ret(grad ? grads_ : params_, n_params_);
  if (name == "grads") return ret(grads_, n_params_);
  if (name == "w_tok") return ret(grad ? A.g_w_tok : A.w_tok, V * d);
  if (name == "w_pos") return ret(grad ? A.g_w_pos : A.w_pos, Tm * d);
  if (name == "lnf_g") return ret(grad ? A.g_lnf_g : A.lnf_g, d);
  if (name == "lnf_b") return ret(grad ? A.g_lnf_b : A.lnf_b, d);
  if (layer < 0 || layer >= (int)cfg_.n_layer) return nullptr;
  const Layer& Y = (*layers_)[layer];
  if (name == "ln1_g") return ret(grad ? Y.g_ln1_g : Y.ln1_g, d);
  if (name == "ln1_b") return ret(grad ? Y.g_ln1_b : Y.ln1_b, d);
  if (name == "ln2_g") return ret(grad ? Y.g_ln2_g : Y.ln2_g, d);
  if (name == "ln2_b") return ret(grad ? Y.g_ln2_b : Y.ln2_b, d);
  if (name == "w_qkv") return ret(grad ? Y.g_w_qkv : Y.w_qkv, 3 * d * d);
  if (name == "w_q") return ret(grad ? Y.g_w_qkv : Y.w_qkv, d * d);
  if (name == "w_k") return ret((grad ? Y.g_w_qkv : Y.w_qkv) + d * d, d * d);
  if (name == "w_v") return ret((grad ? Y.g_w_qkv : Y.w_qkv) + 2 * d * d, d * d);
  if (name == "w_o") return ret(grad ? Y.g_w_o : Y.w_o, d * d);
  if (name == "w_fc") return ret(grad ? Y.g_w_fc : Y.w_fc, F * d);
  if (name == "w_proj") return ret(grad ? Y.g_w_proj : Y.w_proj, d * F);
  return nullptr;
}

void DecoderTransformerGpu::zero_grad() {
  ck(ctx_, aur_memset0(ctx_, grads_, n_params_ * sizeof(float)), "zero_grad");
}

void DecoderTransformerGpu::upload_tokens(const uint32_t* tokens, const uint32_t* targets, uint32_t b,
                                          uint32_t t) {
  const size_t M = (size_t)b * t;
  for (size_t i = 0; i < M; ++i)
    if (tokens[i] >= cfg_.vocab) throw Error("token id out of vocab", AUR_EINVAL);
  ck(ctx_, aur_h2d(ctx_, acts_->tok, tokens, M * 4), "upload tokens");
  if (targets) {
    for (size_t i = 0; i < M; ++i)
      if (targets[i] >= cfg_.vocab) throw Error("target id out of vocab", AUR_EINVAL);
    ck(ctx_, aur_h2d(ctx_, acts_->tgt, targets, M * 4), "upload targets");
  }
}

void DecoderTransformerGpu::encode_forward(uint32_t b, uint32_t t, KvCacheGpu* cache, bool head_all_rows) {
  auto& A = *acts_;
  const int M = (int)(b * t), d = (int)cfg_.d_model, F = (int)cfg_.d_ff, V = (int)cfg_.vocab;
  const int H = (int)cfg_.n_head, dh = d / H;
  ck(ctx_, aur::embed_forward(ctx_, A.w_tok, A.w_pos, A.tok, nullptr, (int)t, A.xs[0], M, d), "embed");
  for (uint32_t l = 0; l < cfg_.n_layer; ++l) {
    Layer& Y = (*layers_)[l];
    ck(ctx_, aur::layer_norm_forward(ctx_, A.xs[l], Y.ln1_g, Y.ln1_b, Y.ln1, Y.mean1, Y.rstd1, M, d, kLnEps),
       "ln1");
    // qkv[M, 3d] = ln1 · [w_q; w_k; w_v]ᵀ  (attention.rs:219 linear_forward ×3)
    ck(ctx_, aur::gemm(ctx_, true, true, Y.ln1, d, Y.w_qkv, d, Y.qkv, 3 * d, M, 3 * d, d, false), "qkv");
    if (cache)
      ck(ctx_, aur::kv_store(ctx_, Y.qkv, d, cache->k_history(l), cache->v_history(l), (int)cache->max_len,
                             nullptr, M, (int)t),
         "kv_store");
    ck(ctx_, aur_mha_fwd_ex(ctx_, Y.qkv, Y.qkv + d, Y.qkv + 2 * d, 3 * d, Y.attn, d, Y.lse, b, t, H, dh),
       "mha_fwd");
    // xmid = x + attn · w_oᵀ  (block.rs:167-172)
    aur::Epilogue resid;
    resid.mode = aur::EPI_RESID;
    resid.R = A.xs[l];
    ck(ctx_, aur::gemm(ctx_, true, true, Y.attn, d, Y.w_o, d, Y.xmid, d, M, d, d, resid), "w_o");
    ck(ctx_, aur::layer_norm_forward(ctx_, Y.xmid, Y.ln2_g, Y.ln2_b, Y.ln2, Y.mean2, Y.rstd2, M, d, kLnEps),
       "ln2");
    // hpre = ln2 · w_fcᵀ, hpost = gelu(hpre)  (ffn.rs:91-105)
    aur::Epilogue ge;
    ge.mode = aur::EPI_GELU;
    ge.C2 = Y.hpost;
    ck(ctx_, aur::gemm(ctx_, true, true, Y.ln2, d, Y.w_fc, d, Y.hpre, F, M, F, d, ge), "w_fc");
    // z = xmid + hpost · w_projᵀ
    aur::Epilogue r2;
    r2.mode = aur::EPI_RESID;
    r2.R = Y.xmid;
    ck(ctx_, aur::gemm(ctx_, true, true, Y.hpost, F, Y.w_proj, F, A.xs[l + 1], d, M, d, F, r2), "w_proj");
  }
  const float* xf = A.xs[cfg_.n_layer];
  ck(ctx_, aur::layer_norm_forward(ctx_, xf, A.lnf_g, A.lnf_b, A.lnf, A.meanf, A.rstdf, M, d, kLnEps), "lnf");
  if (head_all_rows) {
    // tied head: logits = lnf · w_tokᵀ  (embedding.rs:152-169)
    ck(ctx_, aur::gemm(ctx_, true, true, A.lnf, d, A.w_tok, d, A.logits, V, M, V, d, false), "head");
  } else {
    // last position of each sequence only
    ck(ctx_, aur::gather_rows(ctx_, A.lnf, d, (int)t, (int)t - 1, A.last, (int)b, d), "gather last");
    ck(ctx_, aur::gemm(ctx_, true, true, A.last, d, A.w_tok, d, A.logits, V, (int)b, V, d, false), "head");
  }
  (void)F;
}

void DecoderTransformerGpu::encode_backward(uint32_t b, uint32_t t) {
  auto& A = *acts_;
  const int M = (int)(b * t), d = (int)cfg_.d_model, F = (int)cfg_.d_ff, V = (int)cfg_.vocab;
  const int H = (int)cfg_.n_head, dh = d / H;
  float* dlog = A.logits;  // softmax-CE wrote d_logits in place
  // d_h_final = d_logits · w_tok ; g_w_tok += d_logitsᵀ · h_final  (embedding.rs:175-206)
  ck(ctx_, aur::gemm(ctx_, true, false, dlog, V, A.w_tok, d, A.dln, d, M, d, V, false), "head dX");
  ck(ctx_, aur::gemm(ctx_, false, false, dlog, V, A.lnf, d, A.g_w_tok, d, V, d, M, true), "head dW");
  ck(ctx_, aur::layer_norm_backward(ctx_, A.xs[cfg_.n_layer], A.meanf, A.rstdf, A.lnf_g, A.dln, nullptr,
                                    A.dx_a, A.g_lnf_g, A.g_lnf_b, A.ln_ws, M, d),
     "lnf bwd");
  for (int l = (int)cfg_.n_layer - 1; l >= 0; --l) {
    Layer& Y = (*layers_)[l];
    float* dz = A.dx_a;  // gradient w.r.t. this layer's output
    // FFN (ffn.rs:119-149): dh = (dz · w_proj) ⊙ gelu'(hpre); g_w_proj += dzᵀ·hpost
    aur::Epilogue gb;
    gb.mode = aur::EPI_GELU_BWD;
    gb.X = Y.hpre;
    ck(ctx_, aur::gemm(ctx_, true, false, dz, d, Y.w_proj, F, A.dh, F, M, F, d, gb), "proj dX");
    ck(ctx_, aur::gemm(ctx_, false, false, dz, d, Y.hpost, F, Y.g_w_proj, F, d, F, M, true), "proj dW");
    ck(ctx_, aur::gemm(ctx_, true, false, A.dh, F, Y.w_fc, d, A.dln, d, M, d, F, false), "fc dX");
    ck(ctx_, aur::gemm(ctx_, false, false, A.dh, F, Y.ln2, d, Y.g_w_fc, d, F, d, M, true), "fc dW");
    // d_post_attn = dz + LN2'(dln)  (block.rs:207-240)
    ck(ctx_, aur::layer_norm_backward(ctx_, Y.xmid, Y.mean2, Y.rstd2, Y.ln2_g, A.dln, dz, A.dx_b, Y.g_ln2_g,
                                      Y.g_ln2_b, A.ln_ws, M, d),
       "ln2 bwd");
    float* dpa = A.dx_b;
    // MHA (transformer/attention.rs:221-334)
    ck(ctx_, aur::gemm(ctx_, true, false, dpa, d, Y.w_o, d, A.dattn, d, M, d, d, false), "w_o dX");
    ck(ctx_, aur::gemm(ctx_, false, false, dpa, d, Y.attn, d, Y.g_w_o, d, d, d, M, true), "w_o dW");
    // dq, dk, dv stored (not accumulated) into the fused [M, 3d] gradient
    ck(ctx_, aur::mha_bwd_store(ctx_, Y.qkv, Y.qkv + d, Y.qkv + 2 * d, 3 * d, Y.attn, A.dattn, d, Y.lse, A.dqkv,
                                A.dqkv + d, A.dqkv + 2 * d, 3 * d, A.attn_ws, (int)b, (int)t, H, dh),
       "mha_bwd");
    // dx_q + dx_k + dx_v = dqkv · [w_q; w_k; w_v];  g_w_qkv += dqkvᵀ · ln1
    ck(ctx_, aur::gemm(ctx_, true, false, A.dqkv, 3 * d, Y.w_qkv, d, A.dln, d, M, d, 3 * d, false), "qkv dX");
    ck(ctx_, aur::gemm(ctx_, false, false, A.dqkv, 3 * d, Y.ln1, d, Y.g_w_qkv, d, 3 * d, d, M, true),
       "qkv dW");
    // dx = d_post_attn + LN1'(dln)
    ck(ctx_, aur::layer_norm_backward(ctx_, A.xs[l], Y.mean1, Y.rstd1, Y.ln1_g, A.dln, dpa, A.dx_a, Y.g_ln1_g,
                                      Y.g_ln1_b, A.ln_ws, M, d),
       "ln1 bwd");
  }
  (void)V;
}

float DecoderTransformerGpu::train_step_batch(const uint32_t* tokens, const uint32_t* targets, uint32_t b,
                                              uint32_t t, BatchReduction red) {
  if (b == 0 || t == 0) return 0.f;
  if (b > max_batch_ || t > cfg_.seq_len_max) throw Error("train_step_batch: batch/seq too large", AUR_ELIMIT);
  auto& A = *acts_;
  const size_t M = (size_t)b * t;
  for (size_t i = 0; i < M; ++i)
    if (tokens[i] >= cfg_.vocab || targets[i] >= cfg_.vocab)
      throw Error("token or target id out of vocab", AUR_EINVAL);
  hipStream_t st = ctx_->stream;
  // The staging area is free once the previous step's copies out of it ran.
  hip_ck(ctx_, hipEventSynchronize(A.pin_done), "train_step_batch: staging wait");
  std::memcpy(A.pin_tok, tokens, M * 4);
  std::memcpy(A.pin_tgt, targets, M * 4);
  hip_ck(ctx_, hipMemcpyAsync(A.tok, A.pin_tok, M * 4, hipMemcpyHostToDevice, st), "upload tokens");
  hip_ck(ctx_, hipMemcpyAsync(A.tgt, A.pin_tgt, M * 4, hipMemcpyHostToDevice, st), "upload targets");
  encode_forward(b, t, nullptr, true);
  // While the GPU runs the forward: the embedding-gradient scatter plan
  // (rows grouped by token id, ascending; stable within a token), uploaded
  // behind the forward on the same stream, ahead of the backward that reads it.
  int32_t* idx = A.pin_csr_idx;
  std::iota(idx, idx + M, 0);
  std::stable_sort(idx, idx + M, [&](int32_t x, int32_t y) { return tokens[x] < tokens[y]; });
  size_t nuniq = 0;
  for (size_t i = 0; i < M; ++i) {
    if (i == 0 || tokens[idx[i]] != tokens[idx[i - 1]]) {
      A.pin_csr_tok[nuniq] = tokens[idx[i]];
      A.pin_csr_off[nuniq] = (int32_t)i;
      ++nuniq;
    }
  }
  A.pin_csr_off[nuniq] = (int32_t)M;
  auto up = [&](void* dst, const void* src, size_t bytes, const char* what) {
    hip_ck(ctx_, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st), what);
  };
  up(A.csr_tok, A.pin_csr_tok, nuniq * 4, "csr tok");
  up(A.csr_off, A.pin_csr_off, (nuniq + 1) * 4, "csr off");
  up(A.csr_idx, A.pin_csr_idx, M * 4, "csr idx");
  hip_ck(ctx_, hipEventRecord(A.pin_done, st), "train_step_batch: staging event");

  // CE with 1/T per sequence (model.rs:820-858), and for the batch mean the
  // 1/B folded into the same scale; the sum convention keeps 1/T alone.
  const float ce_scale = red == BatchReduction::Sum ? 1.0f / (float)t : 1.0f / ((float)t * b);
  ck(ctx_, aur::softmax_ce(ctx_, A.logits, A.tgt, A.nll, (int)M, (int)cfg_.vocab, ce_scale), "softmax_ce");
  encode_backward(b, t);
  ck(ctx_, aur::embed_backward(ctx_, A.dx_a, (int)b, (int)t, (int)cfg_.d_model, A.csr_tok, A.csr_off, A.csr_idx,
                               (int)nuniq, A.g_w_tok, A.g_w_pos),
     "embed bwd");
  A.nll_host.resize(M);
  ck(ctx_, aur_d2h(ctx_, A.nll_host.data(), A.nll, M * 4), "download nll");
  double s = 0.0;
  for (size_t i = 0; i < M; ++i) s += A.nll_host[i];
  return (float)(s / t);
}

void DecoderTransformerGpu::forward(const uint32_t* tokens, uint32_t b, uint32_t t, float* logits_host) {
  if (b == 0 || t == 0) return;
  if (b > max_batch_ || t > cfg_.seq_len_max) throw Error("forward: batch/seq too large", AUR_ELIMIT);
  upload_tokens(tokens, nullptr, b, t);
  encode_forward(b, t, nullptr, true);
  if (logits_host)
    ck(ctx_, aur_d2h(ctx_, logits_host, acts_->logits, (size_t)b * t * cfg_.vocab * 4), "download logits");
}

void DecoderTransformerGpu::eval_step_batch(const uint32_t* tokens, const uint32_t* targets, uint32_t b,
                                            uint32_t t, float* nll_host) {
  if (b == 0 || t == 0) return;
  if (b > max_batch_ || t > cfg_.seq_len_max) throw Error("eval_step_batch: batch/seq too large", AUR_ELIMIT);
  auto& A = *acts_;
  const size_t M = (size_t)b * t;
  upload_tokens(tokens, targets, b, t);
  encode_forward(b, t, nullptr, true);
  // The logits arena takes the (unused) softmax gradient in place; the NLL
  // rows are exact log-sum-exp minus the target logit, independent of scale.
  ck(ctx_, aur::softmax_ce(ctx_, A.logits, A.tgt, A.nll, (int)M, (int)cfg_.vocab, 1.0f), "softmax_ce");
  ck(ctx_, aur_d2h(ctx_, nll_host, A.nll, M * 4), "download nll");
}

float DecoderTransformerGpu::grad_norm() {
  auto& A = *acts_;
  ck(ctx_, aur::grad_norm(ctx_, grads_, n_params_, INFINITY, A.norm_part, A.stats), "grad norm");
  float nrm = 0.f;
  ck(ctx_, aur_d2h(ctx_, &nrm, A.stats, 4), "download norm");
  return nrm;
}

float DecoderTransformerGpu::clip_grads(float max_norm, bool want_norm) {
  auto& A = *acts_;
  ck(ctx_, aur::grad_norm(ctx_, grads_, n_params_, max_norm, A.norm_part, A.stats), "grad norm");
  ck(ctx_, aur::scale_by(ctx_, grads_, n_params_, A.stats + 1), "clip scale");
  if (!want_norm) return NAN;
  float nrm = 0.f;
  ck(ctx_, aur_d2h(ctx_, &nrm, A.stats, 4), "download norm");
  return nrm;
}

namespace {
// bias_correction (src/optimizer.rs:86-90): 1 − β^t with f32 powi.
inline float powi_f(float b, uint64_t e) {
  float r = 1.0f;
  for (uint64_t i = 0; i < e; ++i) r *= b;
  return r;
}
}  // namespace

void DecoderTransformerGpu::reset_optimizer_state() {
  ck(ctx_, aur_memset0(ctx_, m1_, 2 * n_params_ * sizeof(float)), "zero moments");
  ck(ctx_, aur_memset0(ctx_, mu_, (n_decay_ - (size_t)cfg_.vocab * cfg_.d_model) * sizeof(float)),
     "zero muon momentum");
}

// ------------------------------------------------------------------ Muon
// The matrix parameters (per layer w_q, w_k, w_v = the rows of w_qkv, w_o,
// w_fc, w_proj) occupy [V·d, n_decay) of the flat buffers; the Muon momentum
// buffer mirrors that region.  Newton–Schulz scratch is sized for the
// largest matrix: m = min(rows, cols) = d for every one, n = max ≤ d_ff.
float DecoderTransformerGpu::clip_grads_adamw_subset(float max_norm, bool want_norm) {
  auto& A = *acts_;
  const size_t n_tok = (size_t)cfg_.vocab * cfg_.d_model, n_rest = n_params_ - n_decay_;
  ck(ctx_, aur::grad_norm2(ctx_, grads_, n_tok, grads_ + n_decay_, n_rest, max_norm, A.norm_part, A.stats),
     "subset norm");
  ck(ctx_, aur::scale_by(ctx_, grads_, n_tok, A.stats + 1), "subset clip");
  ck(ctx_, aur::scale_by(ctx_, grads_ + n_decay_, n_rest, A.stats + 1), "subset clip");
  if (!want_norm) return NAN;
  float nrm = 0.f;
  ck(ctx_, aur_d2h(ctx_, &nrm, A.stats, 4), "download norm");
  return nrm;
}

// Muon on every GEMM weight (optimizer.rs:115-305, gpu/transformer.rs:2100-2290),
// batched by matrix shape: the per-matrix work (momentum, Frobenius bound,
// orientation, update) is elementwise, and the 5 Newton–Schulz iterations of
// all matrices of one wide shape m × nn run as strided-batched GEMMs — one
// launch per product for the 4·L square matrices and one for the 2·L FFN
// matrices, instead of 3 small GEMMs per matrix per iteration.  Each matrix's
// arithmetic is the same as one at a time.
void DecoderTransformerGpu::step_muon_hybrid(const MuonConfig& mc, const AdamWConfig& ac) {
  const size_t d = cfg_.d_model, F = cfg_.d_ff, L = cfg_.n_layer, n_tok = (size_t)cfg_.vocab * d;
  struct Mat {
    float* p;
    uint32_t rows, cols;
  };
  // Matrices in the reference's order (gpu/transformer.rs:836-866), rows ×
  // cols as it passes them (w_fc as d × d_ff, w_proj as d_ff × d), grouped by
  // wide shape: square d × d (Q, K, V, O), then min(d,F) × max(d,F) (fc, proj).
  std::vector<Mat> sq, ff;
  for (uint32_t l = 0; l < L; ++l) {
    Layer& Y = (*layers_)[l];
    for (int i = 0; i < 3; ++i) sq.push_back({Y.w_qkv + i * d * d, (uint32_t)d, (uint32_t)d});
    sq.push_back({Y.w_o, (uint32_t)d, (uint32_t)d});
    ff.push_back({Y.w_fc, (uint32_t)d, (uint32_t)F});
    ff.push_back({Y.w_proj, (uint32_t)F, (uint32_t)d});
  }
  const size_t m_ff = std::min(d, F), n_ff = std::max(d, F);
  if (!muon_mem_) {
    const size_t xs = std::max(sq.size() * d * d, ff.size() * m_ff * n_ff);
    const size_t as = std::max(sq.size() * d * d, ff.size() * m_ff * m_ff);
    const size_t floats = 3 * xs + 3 * as + 64;
    ck(ctx_, aur_malloc(ctx_, floats * sizeof(float) + 8 * 256, &muon_mem_), "alloc muon scratch");
    Carver cv{static_cast<char*>(muon_mem_)};
    ns_x_[0] = cv.take<float>(xs);
    ns_x_[1] = cv.take<float>(xs);
    ns_bx_ = cv.take<float>(xs);
    ns_a_ = cv.take<float>(as);
    ns_a2_ = cv.take<float>(as);
    ns_b_ = cv.take<float>(as);
    muon_stats_ = cv.take<float>(64);
  }
  // model.rs:1031-1032: one shared step counter for the AdamW bias correction.
  step += 1;
  const float bc1 = 1.0f - powi_f(ac.beta1, step), bc2 = 1.0f - powi_f(ac.beta2, step);
  // AdamW subset (model.rs:1039-1078): w_tok with decay (embed_lr_mult = 1,
  // the reference default), then w_pos and every LayerNorm γ/β without.
  ck(ctx_, aur::adamw(ctx_, params_, grads_, m1_, m2_, n_tok, n_tok, nullptr, ac.lr, ac.beta1, ac.beta2,
                      ac.eps, ac.weight_decay, bc1, bc2),
     "adamw w_tok");
  ck(ctx_, aur::adamw(ctx_, params_ + n_decay_, grads_ + n_decay_, m1_ + n_decay_, m2_ + n_decay_,
                      n_params_ - n_decay_, 0, nullptr, ac.lr, ac.beta1, ac.beta2, ac.eps, ac.weight_decay,
                      bc1, bc2),
     "adamw undecayed");
  auto& A = *acts_;
  const float a_coef = 3.4445f, b_coef = -4.7750f, c_coef = 2.0315f;
  for (const std::vector<Mat>* grp : {&sq, &ff}) {
    const int nb = (int)grp->size();
    const size_t m = grp == &sq ? d : m_ff, nn = grp == &sq ? d : n_ff, n = m * nn;
    // X0[i] = the momentum update of matrix i, Frobenius-bounded, in wide
    // orientation (optimizer.rs:143-191); ns_bx_ holds a tall one before its
    // transpose.
    for (int i = 0; i < nb; ++i) {
      const Mat& M = (*grp)[i];
      const size_t off = (size_t)(M.p - params_);
      const bool tall = M.rows > M.cols;
      float* u = (tall ? ns_bx_ : ns_x_[0]) + i * n;
      ck(ctx_, aur::muon_momentum(ctx_, grads_ + off, mu_ + (off - n_tok), u, n, mc.momentum, mc.nesterov),
         "muon momentum");
      ck(ctx_, aur::frob_inv(ctx_, u, n, A.norm_part, muon_stats_), "muon frobenius");
      ck(ctx_, aur::scale_by(ctx_, u, n, muon_stats_ + 1), "muon frobenius scale");
      if (tall) ck(ctx_, aur::transpose(ctx_, u, ns_x_[0] + i * n, (int)M.rows, (int)M.cols), "muon load");
    }
    // Newton–Schulz quintic (optimizer.rs:197-239) on the whole group:
    // A = X·Xᵀ, A² = A·A, B = b·A + c·A², X' = a·X + B·X — computed as
    // X' = (a·I + B)·X, one product with no separate pass over X.
    float* x = ns_x_[0];
    const int mi = (int)m, ni = (int)nn;
    for (uint32_t it = 0; it < mc.ns_steps; ++it) {
      float* nxt = (x == ns_x_[0]) ? ns_x_[1] : ns_x_[0];
      ck(ctx_, aur::gemm_batched(ctx_, true, true, x, ni, (long long)n, x, ni, (long long)n, ns_a_, mi,
                                 (long long)(m * m), mi, mi, ni, nb),
         "ns xxt");
      ck(ctx_, aur::gemm_batched(ctx_, true, false, ns_a_, mi, (long long)(m * m), ns_a_, mi, (long long)(m * m),
                                 ns_a2_, mi, (long long)(m * m), mi, mi, mi, nb),
         "ns aa");
      ck(ctx_, aur::ns_combine(ctx_, ns_b_, ns_a_, ns_a2_, a_coef, b_coef, c_coef, mi, nb), "ns combine");
      ck(ctx_, aur::gemm_batched(ctx_, true, false, ns_b_, mi, (long long)(m * m), x, ni, (long long)n, nxt, ni,
                                 (long long)n, mi, ni, mi, nb),
         "ns step");
      x = nxt;
    }
    // p ← p·(1 − lr·wd) − lr·√(max/min)·update, back in the matrix's own
    // orientation (optimizer.rs:241-305).
    const float scale = std::sqrt((float)nn / (float)m);
    for (int i = 0; i < nb; ++i) {
      const Mat& M = (*grp)[i];
      const float* upd = x + i * n;
      if (M.rows > M.cols) {
        ck(ctx_, aur::transpose(ctx_, upd, ns_bx_ + i * n, mi, ni), "muon store");
        upd = ns_bx_ + i * n;
      }
      ck(ctx_, aur::muon_apply(ctx_, M.p, upd, n, mc.lr * scale, mc.lr * mc.weight_decay), "muon apply");
    }
  }
}

void DecoderTransformerGpu::step_adamw(const AdamWConfig& c) {
  step += 1;
  const float bc1 = 1.0f - powi_f(c.beta1, step), bc2 = 1.0f - powi_f(c.beta2, step);
  ck(ctx_, aur::adamw(ctx_, params_, grads_, m1_, m2_, n_params_, n_decay_, nullptr, c.lr, c.beta1, c.beta2,
                      c.eps, c.weight_decay, bc1, bc2),
     "adamw");
}

float DecoderTransformerGpu::clip_and_step_adamw(float max_norm, const AdamWConfig& c, bool want_norm) {
  auto& A = *acts_;
  ck(ctx_, aur::grad_norm(ctx_, grads_, n_params_, max_norm, A.norm_part, A.stats), "grad norm");
  step += 1;
  const float bc1 = 1.0f - powi_f(c.beta1, step), bc2 = 1.0f - powi_f(c.beta2, step);
  ck(ctx_, aur::adamw(ctx_, params_, grads_, m1_, m2_, n_params_, n_decay_, A.stats + 1, c.lr, c.beta1,
                      c.beta2, c.eps, c.weight_decay, bc1, bc2),
     "adamw");
  if (!want_norm) return NAN;
  float nrm = 0.f;
  ck(ctx_, aur_d2h(ctx_, &nrm, A.stats, 4), "download norm");
  return nrm;
}

// ------------------------------------------------------------ state snapshot
// params, then m1 | m2 | Muon momentum, which lie contiguously in
// state_mem_ after the gradients: two device-to-device copies.  The size is
// fixed for the model's lifetime (the momentum is allocated with it).
size_t DecoderTransformerGpu::state_bytes() const {
  return (3 * n_params_ + (n_decay_ - (size_t)cfg_.vocab * cfg_.d_model)) * sizeof(float);
}

void DecoderTransformerGpu::copy_state_to(void* dst, size_t bytes) const {
  if (!dst) throw Error("copy_state_to: null buffer", AUR_EINVAL);
  if (bytes != state_bytes()) throw Error("copy_state_to: buffer size differs from state_bytes()", AUR_EINVAL);
  float* d = static_cast<float*>(dst);
  const size_t n = n_params_ * sizeof(float);
  ck(ctx_, aur_d2d(ctx_, d, params_, n), "snapshot params");
  ck(ctx_, aur_d2d(ctx_, d + n_params_, m1_, bytes - n), "snapshot moments + muon momentum");
}

void DecoderTransformerGpu::copy_state_from(const void* src, size_t bytes) {
  if (!src) throw Error("copy_state_from: null buffer", AUR_EINVAL);
  if (bytes != state_bytes()) throw Error("copy_state_from: buffer size differs from state_bytes()", AUR_EINVAL);
  const float* s = static_cast<const float*>(src);
  const size_t n = n_params_ * sizeof(float);
  ck(ctx_, aur_d2d(ctx_, params_, s, n), "restore params");
  ck(ctx_, aur_d2d(ctx_, m1_, s + n_params_, bytes - n), "restore moments + muon momentum");
}

// ------------------------------------------------------------------ KV cache

KvCacheGpu::KvCacheGpu(DecoderTransformerGpu& model, uint32_t batch_, uint32_t max_len_)
    : batch(batch_), max_len(max_len_), d_model(model.config().d_model), n_layer(model.config().n_layer),
      ctx_(model.ctx()), owner_(&model) {
  const auto& c = model.config();
  if (batch == 0 || max_len == 0 || max_len > c.seq_len_max)
    throw Error("KvCacheGpu: batch > 0 and 0 < max_len <= seq_len_max required", AUR_EINVAL);
  const size_t B = batch, d = d_model, F = c.d_ff, V = c.vocab;
  const size_t hist = (size_t)n_layer * B * max_len * d;
  const size_t scratch = (aur_mha_kv_ws_bytes(batch, c.n_head, max_len) + 3) / 4;
  split = batch <= 64 && d <= 4096;
  if (split) {
    // The decode QKV projection as qkv_parts K-range partials [parts][B][3d]
    // that the attention kernel sums; W_o / W_proj as K-range partials
    // [splits][B][d] that the following LayerNorm sums.
    // (the attention kernel that sums them takes d_head a multiple of 8)
    if ((d / c.n_head) % 8 == 0) qkv_parts = split_override(0, qkv_splits(d), d, 8);
    o_parts = split_override(1, aur::gemm_nt_partials_splits((int)B, (int)d, (int)d), d, 64);
    p_parts = split_override(2, aur::gemm_nt_partials_splits((int)B, (int)d, (int)F), F, 64);
  }
  part_floats_ = (size_t)std::max(o_parts, p_parts) * B * d;
  // x, ln, qkv (3 per part), attn, xmid rows of d per sequence
  const size_t floats =
      2 * hist + B * (d * (4 + 3 * (size_t)qkv_parts) + 2 * F + V) + scratch + part_floats_ + 64;
  bytes_ = floats * 4 + 3 * B * 4 + 40 * 256;
  ck(ctx_, aur_malloc(ctx_, bytes_, &mem_), "KvCacheGpu alloc");
  Carver cv{static_cast<char*>(mem_)};
  k_ = cv.take<float>(hist);
  v_ = cv.take<float>(hist);
  x_ = cv.take<float>(B * d);
  ln_ = cv.take<float>(B * d);
  qkv_ = cv.take<float>((size_t)qkv_parts * 3 * B * d);
  attn_ = cv.take<float>(B * d);
  xmid_ = cv.take<float>(B * d);
  hpre_ = cv.take<float>(B * F);
  hpost_ = cv.take<float>(B * F);
  logits_ = cv.take<float>(B * V);
  scratch_ = cv.take<float>(scratch);
  part_ = cv.take<float>(part_floats_);
  pf_sink_ = cv.take<float>(64);
  pos_ = cv.take<int32_t>(B);
  lens_ = cv.take<int32_t>(B);
  tok_ = cv.take<uint32_t>(B);
  try {
    if (cv.off > bytes_) throw Error("KvCacheGpu: arena overflow", AUR_ENOMEM);
    reset();
  } catch (...) {  // no destructor runs for a constructor that throws
    aur_free(ctx_, mem_);
    mem_ = nullptr;
    throw;
  }
  model.caches_.push_back(this);
}

void KvCacheGpu::drop_graph() {
  if (graph_) {
    aur_sync(ctx_);  // a replay may still be running
    hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_));
    graph_ = nullptr;
  }
}

KvCacheGpu::~KvCacheGpu() {
  if (owner_) {
    auto& v = owner_->caches_;
    v.erase(std::remove(v.begin(), v.end(), this), v.end());
  }
  drop_graph();
  if (mem_) aur_free(ctx_, mem_);
}

void KvCacheGpu::reset() {
  ck(ctx_, aur_memset0(ctx_, mem_, bytes_), "KvCacheGpu reset");
  current_len = 0;
}

void DecoderTransformerGpu::check_cache(const KvCacheGpu& cache) const {
  if (cache.owner_ != this)
    throw Error(cache.owner_ ? "KV cache belongs to another model" : "KV cache's model was destroyed",
                AUR_EINVAL);
}

void DecoderTransformerGpu::prefill_kv(KvCacheGpu& cache, const uint32_t* tokens, uint32_t b, uint32_t t,
                                       float* last_logits) {
  check_cache(cache);
  if (b != cache.batch) throw Error("prefill_kv: batch differs from the cache's", AUR_EINVAL);
  if (t == 0 || t > cache.max_len || b > max_batch_) throw Error("prefill_kv: bad length", AUR_EINVAL);
  cache.reset();
  upload_tokens(tokens, nullptr, b, t);
  encode_forward(b, t, &cache, false);
  auto& A = *acts_;
  const size_t V = cfg_.vocab;
  ck(ctx_, aur_d2d(ctx_, cache.logits_, A.logits, (size_t)b * V * 4), "prefill logits");
  ck(ctx_, aur::argmax_rows(ctx_, cache.logits_, (int)b, (int)V, cache.tok_), "prefill argmax");
  std::vector<int32_t> pos(b, (int32_t)t);
  ck(ctx_, aur_h2d(ctx_, cache.pos_, pos.data(), b * 4), "prefill pos");
  cache.current_len = t;
  ensure_decode_graph(cache);
  if (last_logits) ck(ctx_, aur_d2h(ctx_, last_logits, cache.logits_, (size_t)b * V * 4), "download logits");
}

// One decode step is ~90 small launches: it is captured once per cache as a
// HIP graph (all pointers and shapes are fixed per cache; positions live on
// the device) and replayed, so the host issues one launch per step.  The
// capture is done by prefill_kv, so the first generate_step does not pay for
// it; a cache that was never prefilled captures on first use.
void DecoderTransformerGpu::ensure_decode_graph(KvCacheGpu& cache) {
  if (cache.graph_ || cache.batch > 64) return;
  hipStream_t st = static_cast<hipStream_t>(aur_stream(ctx_));
  if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess)
    throw Error("decode graph: hipStreamBeginCapture failed", AUR_EINVAL);
  try {
    encode_decode_step(cache);
  } catch (...) {
    hipGraph_t g = nullptr;
    hipStreamEndCapture(st, &g);
    if (g) hipGraphDestroy(g);
    throw;
  }
  hipGraph_t g = nullptr;
  if (hipStreamEndCapture(st, &g) != hipSuccess || !g)
    throw Error("decode graph: hipStreamEndCapture failed", AUR_EINVAL);
  hipGraphExec_t ex = nullptr;
  const hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) throw Error("decode graph: hipGraphInstantiate failed", (int)e);
  cache.graph_ = ex;
}

void DecoderTransformerGpu::generate_step_kv(KvCacheGpu& cache, const uint32_t* tokens, float* logits_host,
                                             uint32_t* next_tokens_host) {
  check_cache(cache);
  if (cache.current_len >= cache.max_len) throw Error("generate_step_kv: cache full", AUR_ELIMIT);
  const int B = (int)cache.batch, V = (int)cfg_.vocab;
  if (tokens) {
    for (int i = 0; i < B; ++i)
      if (tokens[i] >= cfg_.vocab) throw Error("token id out of vocab", AUR_EINVAL);
    ck(ctx_, aur_h2d(ctx_, cache.tok_, tokens, (size_t)B * 4), "upload step tokens");
  }
  hipStream_t st = static_cast<hipStream_t>(aur_stream(ctx_));
  if (cache.batch <= 64) {
    ensure_decode_graph(cache);
    const hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(cache.graph_), st);
    if (e != hipSuccess) throw Error(std::string("hipGraphLaunch: ") + hipGetErrorString(e), (int)e);
  } else {
    encode_decode_step(cache);
  }
  cache.current_len += 1;
  if (logits_host) ck(ctx_, aur_d2h(ctx_, logits_host, cache.logits_, (size_t)B * V * 4), "download logits");
  if (next_tokens_host) ck(ctx_, aur_d2h(ctx_, next_tokens_host, cache.tok_, (size_t)B * 4), "download tokens");
}

// Enqueues one decode step for every sequence of `cache`: it reads the input
// token ids and positions from the device (cache.tok_, cache.pos_), leaves the
// logits and their argmax in cache.logits_ / cache.tok_ and advances the
// positions — nothing depends on host values that change between steps.
void DecoderTransformerGpu::encode_decode_step(KvCacheGpu& cache) {
  auto& A = *acts_;
  const int B = (int)cache.batch, d = (int)cfg_.d_model, F = (int)cfg_.d_ff, V = (int)cfg_.vocab;
  const int H = (int)cfg_.n_head, dh = d / H;
  aur::Epilogue store;
  // The two N = d projections (W_o, W_proj) have the fewest output columns:
  // with B ≤ 64 rows they are split into K ranges whose partial products the
  // following LayerNorm sums (with the residual add) — more blocks in flight
  // and no separate reduction launch.
  const bool split = cache.split;
  const int s_o = cache.o_parts, s_p = cache.p_parts;
  // h = w_tok[tok] + w_pos[pos]  (kv_cache.rs:103-115), lens = pos + 1 for
  // the attention below, and the first block's LayerNorm of h (one launch
  // up to the row-resident kernel's d <= 4096, else two)
  if (d <= 4096) {
    ck(ctx_, aur::embed_layer_norm(ctx_, A.w_tok, A.w_pos, cache.tok_, cache.pos_, cache.x_,
                                   (*layers_)[0].ln1_g, (*layers_)[0].ln1_b, cache.ln_, cache.lens_, B, d, kLnEps),
       "embed + ln1");
  } else {
    ck(ctx_, aur::embed_forward(ctx_, A.w_tok, A.w_pos, cache.tok_, cache.pos_, 1, cache.x_, B, d, cache.lens_),
       "embed");
    ck(ctx_, aur::layer_norm_forward(ctx_, cache.x_, (*layers_)[0].ln1_g, (*layers_)[0].ln1_b, cache.ln_, nullptr,
                                     nullptr, B, d, kLnEps),
       "ln1");
  }
  // Attention is launched for lengths up to max_len (keys past a sequence's
  // length are skipped on the device), so the launch shape is the same for
  // every step.
  const int t_max = (int)cache.max_len;
  for (uint32_t l = 0; l < cfg_.n_layer; ++l) {
    Layer& Y = (*layers_)[l];
    // block_step (kv_cache.rs:147-245) for B sequences at once
    if (split && l > 0)  // x = xmid + proj partials of the previous layer
      ck(ctx_, aur::layer_norm_forward_sum(ctx_, cache.xmid_, cache.part_, s_p, cache.x_, Y.ln1_g, Y.ln1_b,
                                           cache.ln_, B, d, kLnEps),
         "ln1");
    else if (l > 0)
      ck(ctx_, aur::layer_norm_forward(ctx_, cache.x_, Y.ln1_g, Y.ln1_b, cache.ln_, nullptr, nullptr, B, d,
                                       kLnEps),
         "ln1");
    // qkv as K-range partials that the attention kernel sums: short K ranges
    // keep the X bytes each CU reads below its weight bytes
    if (cache.qkv_parts > 1)
      ck(ctx_, aur::gemm_nt_partials(ctx_, cache.ln_, d, Y.w_qkv, d, cache.qkv_, B, 3 * d, d, cache.qkv_parts),
         "qkv");
    else
      ck(ctx_, aur::gemm(ctx_, true, true, cache.ln_, d, Y.w_qkv, d, cache.qkv_, 3 * d, B, 3 * d, d, store),
         "qkv");
    // attention of the new query over history + the new row, which the
    // kernel also appends to the history (kv_cache.rs:169-179); its extra
    // blocks pull the following GEMMs' weights into the L2 of the XCDs whose
    // blocks will read them
    aur::L2Prefetch pf;
    if (const char* env = std::getenv("AUR_DEC_PREFETCH")) {
      const char* nb = std::getenv("AUR_DEC_PF_BLOCKS");
      pf.blocks_per_xcd = nb ? std::atoi(nb) : 32;
      pf.sink = cache.pf_sink_;
      auto add = [&](const float* w, int rows, int row_floats, int group) {
        if (pf.nmat < 3 && (rows / group) % 8 == 0) {
          pf.ptr[pf.nmat] = w;
          pf.rows[pf.nmat] = rows;
          pf.row_floats[pf.nmat] = row_floats;
          pf.group[pf.nmat] = group;
          ++pf.nmat;
        }
      };
      for (const char* c = env; *c; ++c) {
        if (*c == 'o') add(Y.w_o, d, d, split ? 64 : 16);  // stream_partials: 64 columns per block
        if (*c == 'f') add(Y.w_fc, F, d, 16);              // skinny: 16 columns per block
        if (*c == 'p') add(Y.w_proj, d, F, split ? 64 : 16);
      }
    }
    if (dh % 8 == 0) {
      ck(ctx_, aur::mha_kv_batched(ctx_, cache.qkv_, 3 * d, cache.k_history(l), cache.v_history(l), cache.attn_,
                                   cache.scratch_, cache.lens_, t_max, B, H, dh, (int)cache.max_len,
                                   cache.qkv_ + d, cache.qkv_ + 2 * d, cache.qkv_parts, (size_t)B * 3 * d, &pf),
         "mha_kv");
    } else {
      // other d_head: the new K/V rows appended at each sequence's position
      // first, then the generic KV kernel over the history
      ck(ctx_, aur::kv_store(ctx_, cache.qkv_, d, cache.k_history(l), cache.v_history(l), (int)cache.max_len,
                             cache.pos_, B, 1),
         "kv_store");
      ck(ctx_, aur::mha_kv_batched(ctx_, cache.qkv_, 3 * d, cache.k_history(l), cache.v_history(l), cache.attn_,
                                   cache.scratch_, cache.lens_, t_max, B, H, dh, (int)cache.max_len, nullptr,
                                   nullptr, 1, 0, nullptr),
         "mha_kv");
    }
    if (split) {
      ck(ctx_, aur::gemm_nt_partials(ctx_, cache.attn_, d, Y.w_o, d, cache.part_, B, d, d, s_o), "w_o");
      ck(ctx_, aur::layer_norm_forward_sum(ctx_, cache.x_, cache.part_, s_o, cache.xmid_, Y.ln2_g, Y.ln2_b,
                                           cache.ln_, B, d, kLnEps),
         "ln2");
    } else {
      aur::Epilogue resid;
      resid.mode = aur::EPI_RESID;
      resid.R = cache.x_;
      ck(ctx_, aur::gemm(ctx_, true, true, cache.attn_, d, Y.w_o, d, cache.xmid_, d, B, d, d, resid), "w_o");
      ck(ctx_, aur::layer_norm_forward(ctx_, cache.xmid_, Y.ln2_g, Y.ln2_b, cache.ln_, nullptr, nullptr, B, d,
                                       kLnEps),
         "ln2");
    }
    aur::Epilogue ge;
    ge.mode = aur::EPI_GELU;
    ge.C2 = cache.hpost_;
    ck(ctx_, aur::gemm(ctx_, true, true, cache.ln_, d, Y.w_fc, d, cache.hpre_, F, B, F, d, ge), "w_fc");
    if (split) {
      ck(ctx_, aur::gemm_nt_partials(ctx_, cache.hpost_, F, Y.w_proj, F, cache.part_, B, d, F, s_p), "w_proj");
    } else {
      aur::Epilogue r2;
      r2.mode = aur::EPI_RESID;
      r2.R = cache.xmid_;
      ck(ctx_, aur::gemm(ctx_, true, true, cache.hpost_, F, Y.w_proj, F, cache.x_, d, B, d, F, r2), "w_proj");
    }
  }
  if (split)
    ck(ctx_, aur::layer_norm_forward_sum(ctx_, cache.xmid_, cache.part_, s_p, cache.x_, A.lnf_g, A.lnf_b,
                                         cache.ln_, B, d, kLnEps),
       "lnf");
  else
    ck(ctx_, aur::layer_norm_forward(ctx_, cache.x_, A.lnf_g, A.lnf_b, cache.ln_, nullptr, nullptr, B, d,
                                     kLnEps),
       "lnf");
  ck(ctx_, aur::gemm(ctx_, true, true, cache.ln_, d, A.w_tok, d, cache.logits_, V, B, V, d, store), "head");
  ck(ctx_, aur::argmax_rows(ctx_, cache.logits_, B, V, cache.tok_, cache.pos_), "argmax");
}

}  // namespace aurora

// ---------------------------------------------------------------- C ABI
using aurora::DecoderTransformerGpu;
using aurora::KvCacheGpu;

struct aur_model {
  DecoderTransformerGpu* m;
};
struct aur_kv_cache {
  KvCacheGpu* c;
  aur_ctx* ctx;  // the context of the model it was created from (which may be gone)
};

namespace {
template <class F>
int guard(aur_ctx* ctx, F&& f) {
  if (ctx) aur::bind_device(ctx);  // the model's GPU, whichever device the thread had current
  try {
    f();
    return 0;
  } catch (const aurora::Error& e) {  // ctx == nullptr: the library-wide slot of aur_last_error(NULL)
    return aur::set_error(ctx, e.code ? e.code : AUR_EINVAL, "%s", e.what());
  } catch (const std::exception& e) {
    return aur::set_error(ctx, AUR_EINVAL, "%s", e.what());
  }
}
}  // namespace

extern "C" {

int aur_model_create(aur_ctx* ctx, const aur_model_config* cfg, uint32_t max_batch, aur_model** out) {
  AUR_CHECK_CTX(ctx);
  if (!cfg || !out) return aur::set_error(ctx, AUR_EINVAL, "aur_model_create: null argument");
  *out = nullptr;
  return guard(ctx, [&] {
    aurora::TransformerConfig c{cfg->vocab, cfg->d_model, cfg->n_layer, cfg->n_head, cfg->d_ff, cfg->seq_len_max};
    auto* m = new aur_model{new DecoderTransformerGpu(ctx, c, max_batch)};
    *out = m;
  });
}

int aur_model_destroy(aur_model* m) {
  if (!m) return 0;
  delete m->m;
  delete m;
  return 0;
}

int aur_model_tensor(aur_model* m, const char* name, int32_t layer, int32_t grad, float** ptr, size_t* len) {
  if (!m || !name || !ptr) return AUR_EINVAL;
  float* p = m->m->tensor(name, layer, grad != 0, len);
  *ptr = p;
  if (!p) return aur::set_error(m->m->ctx(), AUR_EINVAL, "aur_model_tensor: unknown tensor %s[%d]", name, layer);
  return 0;
}

int aur_model_zero_grad(aur_model* m) {
  if (!m) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] { m->m->zero_grad(); });
}

int aur_model_step_muon_hybrid(aur_model* m, float muon_lr, float momentum, int32_t nesterov, float muon_wd,
                               uint32_t ns_steps, float lr, float beta1, float beta2, float eps,
                               float weight_decay) {
  if (!m) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] {
    aurora::MuonConfig mc;
    mc.lr = muon_lr;
    mc.momentum = momentum;
    mc.nesterov = nesterov != 0;
    mc.weight_decay = muon_wd;
    mc.ns_steps = ns_steps;
    aurora::AdamWConfig ac;
    ac.lr = lr;
    ac.beta1 = beta1;
    ac.beta2 = beta2;
    ac.eps = eps;
    ac.weight_decay = weight_decay;
    m->m->step_muon_hybrid(mc, ac);
  });
}

int aur_model_clip_grads_adamw_subset(aur_model* m, float max_norm, float* norm) {
  if (!m) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] {
    const float n = m->m->clip_grads_adamw_subset(max_norm, norm != nullptr);
    if (norm) *norm = n;
  });
}

int aur_checkpoint_peek(const char* path, aur_model_config* cfg, uint32_t* flags, uint32_t* epoch,
                        uint64_t* step) {
  return guard(nullptr, [&] {
    const aurora::CheckpointHeader h = aurora::read_checkpoint_header(path);
    if (cfg) *cfg = aur_model_config{h.cfg.vocab, h.cfg.d_model, h.cfg.n_layer, h.cfg.n_head, h.cfg.d_ff,
                                     h.cfg.seq_len_max};
    if (flags) *flags = h.flags;
    if (epoch) *epoch = h.epoch;
    if (step) *step = h.step;
  });
}

int aur_model_load_checkpoint(aur_model* m, const char* path, uint32_t* epoch, uint64_t* step) {
  if (!m) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] {
    const aurora::CheckpointHeader h = m->m->load_checkpoint(path);
    if (epoch) *epoch = h.epoch;
    if (step) *step = h.step;
  });
}

int aur_model_save_checkpoint(aur_model* m, const char* path, uint32_t epoch, uint64_t step) {
  if (!m) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] { m->m->save_checkpoint(path, epoch, step); });
}

int aur_model_train_step_batch(aur_model* m, const uint32_t* tokens, const uint32_t* targets, uint32_t b,
                               uint32_t t, float* loss_sum) {
  return aur_model_train_step_batch_ex(m, tokens, targets, b, t, AUR_BATCH_MEAN, loss_sum);
}

int aur_model_train_step_batch_ex(aur_model* m, const uint32_t* tokens, const uint32_t* targets, uint32_t b,
                                  uint32_t t, uint32_t reduction, float* loss_sum) {
  if (!m || !tokens || !targets) return AUR_EINVAL;
  if (reduction != AUR_BATCH_MEAN && reduction != AUR_BATCH_SUM)
    return aur::set_error(m->m->ctx(), AUR_EINVAL, "aur_model_train_step_batch_ex: reduction %u", reduction);
  return guard(m->m->ctx(), [&] {
    float l = m->m->train_step_batch(tokens, targets, b, t, static_cast<aurora::BatchReduction>(reduction));
    if (loss_sum) *loss_sum = l;
  });
}

int aur_model_grad_norm(aur_model* m, float* norm) {
  if (!m || !norm) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] { *norm = m->m->grad_norm(); });
}

int aur_model_state_bytes(aur_model* m, size_t* bytes) {
  if (!m || !bytes) return AUR_EINVAL;
  *bytes = m->m->state_bytes();
  return 0;
}

int aur_model_state_save(aur_model* m, void* dst, size_t bytes, uint64_t* step) {
  if (!m || !dst) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] {
    m->m->copy_state_to(dst, bytes);
    if (step) *step = m->m->step;
  });
}

int aur_model_state_load(aur_model* m, const void* src, size_t bytes, uint64_t step) {
  if (!m || !src) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] {
    m->m->copy_state_from(src, bytes);
    m->m->step = step;
  });
}

int aur_model_forward(aur_model* m, const uint32_t* tokens, uint32_t b, uint32_t t, float* logits) {
  if (!m || !tokens) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] { m->m->forward(tokens, b, t, logits); });
}

int aur_model_eval_step_batch(aur_model* m, const uint32_t* tokens, const uint32_t* targets, uint32_t b,
                              uint32_t t, float* nll) {
  if (!m || !tokens || !targets || !nll) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] { m->m->eval_step_batch(tokens, targets, b, t, nll); });
}

int aur_model_clip_grads(aur_model* m, float max_norm, float* norm) {
  if (!m) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] {
    float n = m->m->clip_grads(max_norm, norm != nullptr);
    if (norm) *norm = n;
  });
}

int aur_model_step_adamw(aur_model* m, float lr, float beta1, float beta2, float eps, float weight_decay) {
  if (!m) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] { m->m->step_adamw(aurora::AdamWConfig{lr, beta1, beta2, eps, weight_decay}); });
}

int aur_model_clip_step_adamw(aur_model* m, float max_norm, float lr, float beta1, float beta2, float eps,
                              float weight_decay, float* norm) {
  if (!m) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] {
    float n = m->m->clip_and_step_adamw(max_norm, aurora::AdamWConfig{lr, beta1, beta2, eps, weight_decay},
                                        norm != nullptr);
    if (norm) *norm = n;
  });
}

int aur_kv_cache_create(aur_model* m, uint32_t batch, uint32_t max_len, aur_kv_cache** out) {
  if (!m || !out) return AUR_EINVAL;
  *out = nullptr;
  return guard(m->m->ctx(), [&] { *out = new aur_kv_cache{new KvCacheGpu(*m->m, batch, max_len), m->m->ctx()}; });
}

int aur_kv_cache_reset(aur_kv_cache* c) {
  if (!c) return AUR_EINVAL;
  return guard(c->ctx, [&] { c->c->reset(); });
}

int aur_kv_cache_destroy(aur_kv_cache* c) {
  if (!c) return 0;
  delete c->c;
  delete c;
  return 0;
}

int aur_kv_cache_len(aur_kv_cache* c, uint32_t* len) {
  if (!c || !len) return AUR_EINVAL;
  *len = c->c->current_len;
  return 0;
}

int aur_kv_cache_history(aur_kv_cache* c, uint32_t layer, float** k, float** v) {
  if (!c || !k || !v || layer >= c->c->n_layer) return AUR_EINVAL;
  *k = c->c->k_history(layer);
  *v = c->c->v_history(layer);
  return 0;
}

int aur_model_prefill_kv(aur_model* m, aur_kv_cache* c, const uint32_t* tokens, uint32_t b, uint32_t t,
                         float* last_logits) {
  if (!m || !c || !tokens) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] { m->m->prefill_kv(*c->c, tokens, b, t, last_logits); });
}

int aur_model_generate_step(aur_model* m, aur_kv_cache* c, const uint32_t* tokens, float* logits,
                            uint32_t* next_tokens) {
  if (!m || !c) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] { m->m->generate_step_kv(*c->c, tokens, logits, next_tokens); });
}

int aur_model_generate_greedy(aur_model* m, aur_kv_cache* c, uint32_t n_steps, uint32_t* out_tokens) {
  if (!m || !c) return AUR_EINVAL;
  return guard(m->m->ctx(), [&] {
    const uint32_t B = c->c->batch;
    for (uint32_t s = 0; s < n_steps; ++s)
      m->m->generate_step_kv(*c->c, nullptr, nullptr, out_tokens ? out_tokens + (size_t)s * B : nullptr);
  });
}

}  // extern "C"
