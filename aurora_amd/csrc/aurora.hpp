// aurora.hpp — C++ host interface over libaurora_hip.so, shaped like the
// reference crate's `aurora::gpu` surface (src/gpu/mod.rs:40-63):
//
//   GpuContext                 src/gpu/context.rs:5-75     (one device, one stream)
//   GpuBuffer<T>               src/gpu/buffers.rs:14-192   (caller-owned device memory)
//   GemmKernel                 src/gpu/matmul.rs:230-356   C = A·B
//   GemmTransposeBKernel       src/gpu/matmul.rs:358-409   C = A·Bᵀ
//   OuterProductAccumKernel    src/gpu/reduce.rs:125-241   dest += dYᵀ·X
//   CausalMhaForwardKernel     src/gpu/attention.rs:346-483
//   CausalMhaBackwardKernel    src/gpu/attention.rs:485-801
//   MhaKvCacheKernel           src/gpu/kv_cache.rs:366-466
//   DecoderTransformerGpu      src/gpu/transformer.rs:32-116 (train step, KV decode)
//   KvCacheGpu                 src/gpu/kv_cache.rs:21-92
//
// Kernel structs keep the reference's argument order and its contract:
// `dispatch_into` only enqueues on the context's stream, buffers belong to
// the caller.  GpuContext construction is the one fallible step of the
// reference (GpuContext::new() -> Result); here every failure throws
// aurora::Error carrying aur_last_error's message.
#pragma once

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/aurora_hip.h"

namespace aurora {

class Error : public std::runtime_error {
 public:
  Error(const std::string& what, int code) : std::runtime_error(what), code(code) {}
  int code;
};

inline void check(const aur_ctx* ctx, int rc, const char* what) {
  if (rc != 0) throw Error(std::string(what) + ": " + aur_last_error(ctx), rc);
}

class GpuContext {
 public:
  explicit GpuContext(int device = 0) {
    int rc = aur_init(device, &ctx_);
    if (rc != 0) throw Error(std::string("GpuContext::new: ") + aur_last_error(nullptr), rc);
  }
  ~GpuContext() { aur_destroy(ctx_); }
  GpuContext(const GpuContext&) = delete;
  GpuContext& operator=(const GpuContext&) = delete;
  aur_ctx* raw() const { return ctx_; }
  void sync() const { check(ctx_, aur_sync(ctx_), "aur_sync"); }

 private:
  aur_ctx* ctx_ = nullptr;
};

template <class T>
class GpuBuffer {
 public:
  GpuBuffer(const GpuContext& ctx, size_t len) : ctx_(ctx.raw()), len_(len) {
    void* p = nullptr;
    check(ctx_, aur_malloc(ctx_, len * sizeof(T) + (len == 0), &p), "GpuBuffer::empty");
    ptr_ = static_cast<T*>(p);
  }
  static GpuBuffer zeros(const GpuContext& ctx, size_t len) {
    GpuBuffer b(ctx, len);
    check(b.ctx_, aur_memset0(b.ctx_, b.ptr_, len * sizeof(T)), "GpuBuffer::zeros");
    return b;
  }
  static GpuBuffer from_slice(const GpuContext& ctx, const std::vector<T>& data) {
    GpuBuffer b(ctx, data.size());
    b.upload(data);
    return b;
  }
  GpuBuffer(GpuBuffer&& o) noexcept : ctx_(o.ctx_), ptr_(o.ptr_), len_(o.len_) { o.ptr_ = nullptr; }
  GpuBuffer(const GpuBuffer&) = delete;
  ~GpuBuffer() {
    if (ptr_) aur_free(ctx_, ptr_);
  }
  void upload(const std::vector<T>& data) {
    if (data.size() > len_) throw Error("GpuBuffer::upload: too long", AUR_EINVAL);
    check(ctx_, aur_h2d(ctx_, ptr_, data.data(), data.size() * sizeof(T)), "GpuBuffer::upload");
  }
  std::vector<T> download() const {
    std::vector<T> out(len_);
    check(ctx_, aur_d2h(ctx_, out.data(), ptr_, len_ * sizeof(T)), "GpuBuffer::download");
    return out;
  }
  T* ptr() const { return ptr_; }
  size_t len() const { return len_; }

 private:
  aur_ctx* ctx_;
  T* ptr_ = nullptr;
  size_t len_;
};

// The kernels read and write exactly the extents their dimensions name; a
// buffer shorter than that is refused here, where its length is known (the
// reference's WGSL had wgpu's bounds-checked buffer access instead — an
// out-of-range access on the GPU faults).
inline void need(const GpuBuffer<float>& b, size_t n, const char* what) {
  if (b.len() < n)
    throw Error(std::string(what) + ": buffer of " + std::to_string(b.len()) + " floats, " +
                    std::to_string(n) + " needed",
                AUR_EINVAL);
}

struct GemmKernel {
  void dispatch_into(const GpuContext& c, const GpuBuffer<float>& a, const GpuBuffer<float>& b,
                     const GpuBuffer<float>& out, uint32_t m, uint32_t n, uint32_t k) const {
    need(a, (size_t)m * k, "GemmKernel a");
    need(b, (size_t)k * n, "GemmKernel b");
    need(out, (size_t)m * n, "GemmKernel c");
    check(c.raw(), aur_gemm_nn(c.raw(), a.ptr(), b.ptr(), out.ptr(), m, n, k), "GemmKernel");
  }
};

struct GemmTransposeBKernel {
  void dispatch_into(const GpuContext& c, const GpuBuffer<float>& a, const GpuBuffer<float>& b,
                     const GpuBuffer<float>& out, uint32_t m, uint32_t n, uint32_t k) const {
    need(a, (size_t)m * k, "GemmTransposeBKernel a");
    need(b, (size_t)n * k, "GemmTransposeBKernel b");
    need(out, (size_t)m * n, "GemmTransposeBKernel c");
    check(c.raw(), aur_gemm_nt(c.raw(), a.ptr(), b.ptr(), out.ptr(), m, n, k), "GemmTransposeBKernel");
  }
};

struct OuterProductAccumKernel {
  void dispatch_into(const GpuContext& c, const GpuBuffer<float>& x, const GpuBuffer<float>& d_y,
                     const GpuBuffer<float>& dest, uint32_t d_out, uint32_t d_in, uint32_t t) const {
    need(x, (size_t)t * d_in, "OuterProductAccumKernel x");
    need(d_y, (size_t)t * d_out, "OuterProductAccumKernel d_y");
    need(dest, (size_t)d_out * d_in, "OuterProductAccumKernel dest");
    check(c.raw(), aur_outer_accum(c.raw(), x.ptr(), d_y.ptr(), dest.ptr(), d_out, d_in, t),
          "OuterProductAccumKernel");
  }
};

struct CausalMhaForwardKernel {
  // `lse` [b, n_head, t] takes the reference's `probs` slot.
  void dispatch_into(const GpuContext& c, const GpuBuffer<float>& q, const GpuBuffer<float>& k,
                     const GpuBuffer<float>& v, const GpuBuffer<float>& out, const GpuBuffer<float>& lse,
                     uint32_t t, uint32_t n_head, uint32_t d_head, uint32_t b = 1) const {
    const size_t act = (size_t)b * t * n_head * d_head;
    for (const GpuBuffer<float>* x : {&q, &k, &v, &out}) need(*x, act, "CausalMhaForwardKernel q/k/v/out");
    need(lse, (size_t)b * n_head * t, "CausalMhaForwardKernel lse");
    check(c.raw(), aur_mha_fwd(c.raw(), q.ptr(), k.ptr(), v.ptr(), out.ptr(), lse.ptr(), b, t, n_head, d_head),
          "CausalMhaForwardKernel");
  }
};

struct CausalMhaBackwardKernel {
  static size_t workspace_len(uint32_t t, uint32_t n_head, uint32_t b = 1) {
    return (aur_mha_bwd_ws_bytes(b, t, n_head) + 3) / 4;
  }
  // dq, dk, dv accumulate; the caller zeroes them first (attention.rs:575-578).
  void dispatch_into(const GpuContext& c, const GpuBuffer<float>& q, const GpuBuffer<float>& k,
                     const GpuBuffer<float>& v, const GpuBuffer<float>& out, const GpuBuffer<float>& lse,
                     const GpuBuffer<float>& d_out, const GpuBuffer<float>& dq, const GpuBuffer<float>& dk,
                     const GpuBuffer<float>& dv, const GpuBuffer<float>& ws, uint32_t t, uint32_t n_head,
                     uint32_t d_head, uint32_t b = 1) const {
    const size_t act = (size_t)b * t * n_head * d_head;
    for (const GpuBuffer<float>* x : {&q, &k, &v, &out, &d_out, &dq, &dk, &dv})
      need(*x, act, "CausalMhaBackwardKernel q/k/v/out/d_out/dq/dk/dv");
    need(lse, (size_t)b * n_head * t, "CausalMhaBackwardKernel lse");
    need(ws, workspace_len(t, n_head, b), "CausalMhaBackwardKernel workspace");
    check(c.raw(),
          aur_mha_bwd(c.raw(), q.ptr(), k.ptr(), v.ptr(), out.ptr(), lse.ptr(), d_out.ptr(), dq.ptr(),
                      dk.ptr(), dv.ptr(), ws.ptr(), b, t, n_head, d_head),
          "CausalMhaBackwardKernel");
  }
};

struct MhaKvCacheKernel {
  static size_t scratch_len(uint32_t n_head, uint32_t max_len, uint32_t b = 1) {
    return (aur_mha_kv_ws_bytes(b, n_head, max_len) + 3) / 4;
  }
  void dispatch_into(const GpuContext& c, const GpuBuffer<float>& q_new, const GpuBuffer<float>& k_history,
                     const GpuBuffer<float>& v_history, const GpuBuffer<float>& out,
                     const GpuBuffer<float>& scratch, uint32_t t_total, uint32_t n_head, uint32_t d_head,
                     uint32_t max_len) const {
    const size_t d = (size_t)n_head * d_head;
    need(q_new, d, "MhaKvCacheKernel q_new");
    need(out, d, "MhaKvCacheKernel out");
    need(k_history, (size_t)max_len * d, "MhaKvCacheKernel k_history");
    need(v_history, (size_t)max_len * d, "MhaKvCacheKernel v_history");
    need(scratch, scratch_len(n_head, max_len), "MhaKvCacheKernel scratch");
    check(c.raw(),
          aur_mha_kv_step(c.raw(), q_new.ptr(), k_history.ptr(), v_history.ptr(), out.ptr(), scratch.ptr(),
                          t_total, n_head, d_head, max_len),
          "MhaKvCacheKernel");
  }
};

// ----------------------------------------------------------------- model

// src/transformer/model.rs:24-127 (the fields this backend supports: the
// plain pre-LN GPT of every BASELINE config; optional features are off).
struct TransformerConfig {
  uint32_t vocab, d_model, n_layer, n_head, d_ff, seq_len_max;
};

// src/optimizer.rs:20-38
struct AdamWConfig {
  float lr = 6e-4f, beta1 = 0.9f, beta2 = 0.95f, eps = 1e-8f, weight_decay = 0.1f;
};

// src/optimizer.rs:94-113
struct MuonConfig {
  float lr = 0.02f, momentum = 0.95f;
  bool nesterov = true;
  float weight_decay = 0.0f;
  uint32_t ns_steps = 5;
};

class KvCacheGpu;

// Header of an AURORA05/06/07 checkpoint (src/checkpoint.rs:9-49).
struct CheckpointHeader {
  int version = 0;  // 5, 6 or 7
  TransformerConfig cfg;
  uint32_t flags = 0;  // rope, rmsnorm, relu2, qk_norm, untied_head, swiglu, layerscale, parallel, diff_attn, head_bias
  float softcap = 0.f;
  uint32_t canon_kernel = 0, sink_tokens = 0, epoch = 0;
  uint64_t step = 0;
};
CheckpointHeader read_checkpoint_header(const char* path);
CheckpointHeader read_checkpoint_header(std::FILE* f);

// How train_step_batch combines the B per-sequence gradients (each of a
// mean-over-T cross-entropy): Sum is the reference GPU model's convention
// (src/gpu/transformer.rs:1555-1559; its trainer scales the clip threshold by
// B, examples/aurora_train.rs:1046-1051), Mean the CPU trainer's
// grads.scale(1/B) (examples/aurora_train.rs:840-846).
enum class BatchReduction : uint32_t { Mean = AUR_BATCH_MEAN, Sum = AUR_BATCH_SUM };

// The reference's DecoderTransformerGpu at M = B·T rows: B sequences of
// length T run through every GEMM together (the reference serialises them,
// one sequence per GEMM).
class DecoderTransformerGpu {
 public:
  DecoderTransformerGpu(aur_ctx* ctx, const TransformerConfig& cfg, uint32_t max_batch);
  ~DecoderTransformerGpu();
  DecoderTransformerGpu(const DecoderTransformerGpu&) = delete;
  DecoderTransformerGpu& operator=(const DecoderTransformerGpu&) = delete;

  const TransformerConfig& config() const { return cfg_; }
  aur_ctx* ctx() const { return ctx_; }
  uint64_t step = 0;  // AdamW step counter (model.rs step)

  // Device tensor `name` (w_tok, w_pos, ln1_g, ln1_b, w_q, w_k, w_v, w_qkv,
  // w_o, ln2_g, ln2_b, w_fc, w_proj, lnf_g, lnf_b, params, grads) of `layer`;
  // grad selects the gradient twin.  Returns nullptr for an unknown name.
  float* tensor(const std::string& name, int layer, bool grad, size_t* n) const;
  size_t param_count() const { return n_params_; }

  void zero_grad();
  // Forward + softmax-CE + backward for b sequences of length t; gradients
  // accumulate, combined over the batch as `red` says.  Returns
  // Σ_b mean_t NLL_b (src/gpu/transformer.rs:1571-1615).
  float train_step_batch(const uint32_t* tokens, const uint32_t* targets, uint32_t b, uint32_t t,
                         BatchReduction red = BatchReduction::Mean);
  // Forward only; logits [b·t, vocab] to the host if non-null.
  void forward(const uint32_t* tokens, uint32_t b, uint32_t t, float* logits_host);
  // Forward + softmax-CE with loss scale 1 and no backward: per-token NLL in
  // nats for b windows of length t into nll_host [b·t] (window-major).
  // Parameters, gradients and optimizer moments are not touched
  // (src/gpu/transformer.rs:1723-1811).
  void eval_step_batch(const uint32_t* tokens, const uint32_t* targets, uint32_t b, uint32_t t,
                       float* nll_host);
  // grad_norm (src/gpu/transformer.rs:1263): global L2 norm over all grads.
  float grad_norm();
  // model.rs:1011-1017: global L2 norm over all grads, scaled in place when
  // above max_norm; returns the pre-clip norm, or NaN without the host read
  // when want_norm is false (src/gpu/transformer.rs:2294 want_norm).
  float clip_grads(float max_norm, bool want_norm = true);
  // model.rs:926-1009 (decay on w_tok, Q/K/V/O, fc, proj; none on LN, w_pos).
  void step_adamw(const AdamWConfig& cfg);
  // clip_grads + step_adamw without the separate scaling pass.
  float clip_and_step_adamw(float max_norm, const AdamWConfig& cfg, bool want_norm = true);

  // Muon hybrid (model.rs:1023-1090, gpu/transformer.rs:2052-2291): AdamW on
  // the embeddings and LayerNorm γ/β, Muon (momentum → Frobenius bound →
  // ns_steps quintic Newton–Schulz on the GEMMs → √(max/min) scale) on every
  // Q/K/V/O/fc/proj matrix.  The Muon momentum buffers are allocated on the
  // first call.
  void step_muon_hybrid(const MuonConfig& muon, const AdamWConfig& adam);
  // model.rs:1101-1107: L2 norm over the AdamW subset only, which is scaled
  // to max_norm when above it; returns the pre-clip norm (NaN when
  // want_norm is false: no host read).
  float clip_grads_adamw_subset(float max_norm, bool want_norm = true);

  // snapshot_state / refresh_state / restore_state (src/gpu/transformer.rs:
  // 1152-1240): the persistent state — parameters, both AdamW moments and
  // the Muon momentum (allocated with the model, as the reference's mu
  // buffers are, so the size never changes) — copied device-to-device into
  // or out of a caller-owned buffer of `bytes` bytes, which must equal
  // state_bytes() (AUR_EINVAL otherwise).  The optimizer step counter
  // travels separately (`step`).
  size_t state_bytes() const;
  void copy_state_to(void* dst, size_t bytes) const;
  void copy_state_from(const void* src, size_t bytes);

  // Zero the optimizer state (AdamW moments, Muon momentum) — a fresh optimizer.
  void reset_optimizer_state();
  // checkpoint.rs save / load (AURORA07 writes; AURORA05-07 reads).  load
  // requires this model's dimensions, refuses optional features the
  // backend lacks (AUR_ELIMIT), resets the optimizer state and sets `step`.
  void save_checkpoint(const char* path, uint32_t epoch, uint64_t step) const;
  CheckpointHeader load_checkpoint(const char* path);

  // KV decode (src/gpu/transformer.rs:2374-2640, batched).  A cache serves
  // only the model it was created from (its captured decode step holds that
  // model's weight pointers); other models get AUR_EINVAL.
  void prefill_kv(KvCacheGpu& cache, const uint32_t* tokens, uint32_t b, uint32_t t, float* last_logits);
  void generate_step_kv(KvCacheGpu& cache, const uint32_t* tokens, float* logits_host,
                        uint32_t* next_tokens_host);

 private:
  friend class KvCacheGpu;
  struct Layer;
  struct Acts;
  void encode_forward(uint32_t b, uint32_t t, KvCacheGpu* cache, bool head_all_rows);
  void encode_decode_step(KvCacheGpu& cache);
  void ensure_decode_graph(KvCacheGpu& cache);
  void encode_backward(uint32_t b, uint32_t t);
  void upload_tokens(const uint32_t* tokens, const uint32_t* targets, uint32_t b, uint32_t t);
  void check_cache(const KvCacheGpu& cache) const;
  void init();              // the constructor's work
  void release() noexcept;  // frees whatever init() or later calls allocated

  aur_ctx* ctx_;
  TransformerConfig cfg_;
  uint32_t max_batch_;
  size_t n_params_ = 0, n_decay_ = 0;
  void* state_mem_ = nullptr;  // params | grads | m1 | m2
  void* muon_mem_ = nullptr;   // Muon momentum of the matrix region + Newton–Schulz scratch
  // per shape group: ns_x_ / ns_bx_ hold [matrices][m × nn], ns_a_ / ns_a2_ / ns_b_ [matrices][m × m]
  float *mu_ = nullptr, *ns_x_[2] = {nullptr, nullptr}, *ns_bx_ = nullptr;
  float *ns_a_ = nullptr, *ns_a2_ = nullptr, *ns_b_ = nullptr, *muon_stats_ = nullptr;
  void* act_mem_ = nullptr;
  float *params_ = nullptr, *grads_ = nullptr, *m1_ = nullptr, *m2_ = nullptr;
  std::vector<Layer>* layers_ = nullptr;
  Acts* acts_ = nullptr;
  // Live caches created from this model; on destruction they are detached
  // (their decode graphs, which read this model's weights, are dropped).
  std::vector<KvCacheGpu*> caches_;
};

// Per-layer K/V history for a batch of sequences decoded together:
// [n_layer][batch][max_len][d_model] each for K and V, plus the device-side
// positions and decode activations (src/gpu/kv_cache.rs:21-92).  It belongs
// to the model it is created from and must not outlive it in use: once that
// model is destroyed the cache can only be destroyed.
class KvCacheGpu {
 public:
  KvCacheGpu(DecoderTransformerGpu& model, uint32_t batch, uint32_t max_len);
  ~KvCacheGpu();
  KvCacheGpu(const KvCacheGpu&) = delete;
  KvCacheGpu& operator=(const KvCacheGpu&) = delete;
  // Zero all history and positions (kv_cache.rs:76-91).
  void reset();
  uint32_t batch, max_len, d_model, n_layer;
  uint32_t current_len = 0;
  float* k_history(uint32_t layer) const { return k_ + (size_t)layer * batch * max_len * d_model; }
  float* v_history(uint32_t layer) const { return v_ + (size_t)layer * batch * max_len * d_model; }

 private:
  friend class DecoderTransformerGpu;
  void drop_graph();
  aur_ctx* ctx_;
  DecoderTransformerGpu* owner_;  // nullptr once the model is destroyed
  void* mem_ = nullptr;
  float *k_ = nullptr, *v_ = nullptr;
  int32_t *pos_ = nullptr, *lens_ = nullptr;
  uint32_t* tok_ = nullptr;
  float *x_ = nullptr, *ln_ = nullptr, *qkv_ = nullptr, *attn_ = nullptr, *xmid_ = nullptr;
  float *hpre_ = nullptr, *hpost_ = nullptr, *logits_ = nullptr, *scratch_ = nullptr;
  float* part_ = nullptr;  // K-range partial products of the W_o / W_proj decode GEMMs
  float* pf_sink_ = nullptr;  // the L2 prefetch blocks' never-written sink
  size_t part_floats_ = 0;
  int qkv_parts = 1;  // K ranges of the decode QKV projection held in qkv_
  int o_parts = 1, p_parts = 1;  // K ranges of the W_o / W_proj products in part_
  // W_o / W_proj as K-range partials summed by the following LayerNorm
  // (batch <= 64 and d_model <= 4096, the row-resident LayerNorm kernels'
  // limit); otherwise whole products with the residual fused.
  bool split = false;
  size_t bytes_ = 0;
  void* graph_ = nullptr;       // hipGraphExec_t of one decode step, built on first use
};

}  // namespace aurora
