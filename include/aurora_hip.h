/*
 * aurora_hip.h — C ABI of libaurora_hip.so, the MI355X (gfx950) backend for
 * Aurora's matrix-multiply / causal-attention hot path.
 *
 * Conventions (all entry points):
 *   - every function returns int: 0 = success, otherwise a hipError_t value or
 *     one of the AUR_E* codes below; aur_last_error(ctx) gives the message.
 *   - every pointer argument that names a tensor is a DEVICE pointer owned by
 *     the caller (allocated with aur_malloc or any other HIP allocator); the
 *     launchers never allocate tensors.  Tensors are fp32 row-major, token ids
 *     and lengths are 32-bit.
 *   - all work of one context is ordered on that context's single HIP stream;
 *     launchers only enqueue (no host sync) — like the reference's
 *     `dispatch_into`, which only records into a wgpu::CommandEncoder.
 *     aur_d2h and aur_sync are the synchronising calls.
 *   - a context is not thread-safe; callers serialise access to it (the
 *     reference's GpuContext likewise wraps one queue).
 *
 * Weights follow the reference layout [d_out, d_in] (src/attention.rs:162-167),
 * so a forward linear is y = x·Wᵀ (aur_gemm_nt).
 */
#ifndef AURORA_HIP_H
#define AURORA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct aur_ctx aur_ctx;

#define AUR_OK 0
/* Library-level error codes sit above the hipError_t range. */
#define AUR_EINVAL 10001   /* bad argument (shape, null pointer, alignment) */
#define AUR_ENOMEM 10002   /* workspace could not be obtained */
#define AUR_ELIMIT 10003   /* shape exceeds a documented kernel limit */
#define AUR_EIO 10004      /* checkpoint file could not be opened, read or written */

/* ---- context / runtime (replaces src/gpu/context.rs:22-69 GpuContext::new
 *      and src/gpu/buffers.rs:27-191 GpuBuffer) ------------------------- */

/* Create a context on HIP device `device` with one default-priority stream.
 * Mirrors GpuContext::new() -> Result<Self, GpuInitError> (context.rs:22):
 * the only fallible constructor; non-zero when no usable gfx950 device.
 * Every call taking a context (or a model / cache made from one) first makes
 * that context's device current for the calling thread, so a process may
 * drive one context per GPU from one thread. */
int aur_init(int device, aur_ctx** out);
int aur_destroy(aur_ctx* ctx);
/* Message of the last failing call on this context ("" if none). ctx may be
 * NULL, then the message of the last aur_init failure is returned. */
const char* aur_last_error(const aur_ctx* ctx);
/* The context's stream (a hipStream_t) for callers that interoperate. */
void* aur_stream(aur_ctx* ctx);
/* Device name + arch, e.g. "AMD Instinct MI355X gfx950:sramecc+:xnack-". */
int aur_device_info(aur_ctx* ctx, char* buf, size_t len, int* cu_count);

/* Memory: GpuBuffer::{empty,zeros,from_slice,upload,download}
 * (buffers.rs:27-191).  aur_d2h blocks until the copy is done, like
 * GpuBuffer::download (map_async + poll(Wait)). */
int aur_malloc(aur_ctx* ctx, size_t bytes, void** out);
int aur_free(aur_ctx* ctx, void* ptr);
int aur_h2d(aur_ctx* ctx, void* dst, const void* src, size_t bytes);
int aur_d2h(aur_ctx* ctx, void* dst, const void* src, size_t bytes);
int aur_d2d(aur_ctx* ctx, void* dst, const void* src, size_t bytes);
int aur_memset0(aur_ctx* ctx, void* dst, size_t bytes);
int aur_sync(aur_ctx* ctx);

/* Timing on the context's stream (replaces the reference's wgpu
 * timestamp-query GpuProfiler mark/resolve, src/gpu/profiler.rs:13-138).
 * aur_event_elapsed_ms waits for `stop` and returns stop − start in ms. */
int aur_event_create(aur_ctx* ctx, void** ev);
int aur_event_record(aur_ctx* ctx, void* ev);
int aur_event_elapsed_ms(aur_ctx* ctx, void* start, void* stop, float* ms);
int aur_event_destroy(aur_ctx* ctx, void* ev);

/* ---- GEMM family --------------------------------------------------------- */

/* C[m,n] = A[m,k] · B[k,n]   (overwrite).
 * Replaces GemmKernel::dispatch_into(ctx, enc, a, b, c, m, n, k)
 * (src/gpu/matmul.rs:285-321; WGSL GEMM_WGSL matmul.rs:21-120). */
int aur_gemm_nn(aur_ctx* ctx, const float* a, const float* b, float* c,
                uint32_t m, uint32_t n, uint32_t k);

/* C[m,n] = Σ_k A[m,k] · B[n,k]   (overwrite) — every forward linear y = x·Wᵀ
 * and the tied LM head.
 * Replaces GemmTransposeBKernel::dispatch_into(ctx, enc, a, b, c, m, n, k)
 * (src/gpu/matmul.rs:371-383; WGSL matmul.rs:122-219). */
int aur_gemm_nt(aur_ctx* ctx, const float* a, const float* b, float* c,
                uint32_t m, uint32_t n, uint32_t k);

/* dest[d_out,d_in] += Σ_t d_y[t,d_out] · x[t,d_in]   (read-modify-write,
 * deterministic, no atomics: a split over t is reduced in a fixed order).
 * Replaces OuterProductAccumKernel::dispatch_into(ctx, enc, x, d_y, dest,
 * d_out, d_in, t) (src/gpu/reduce.rs:176-207; WGSL reduce.rs:15-115). */
int aur_outer_accum(aur_ctx* ctx, const float* x, const float* d_y, float* dest,
                    uint32_t d_out, uint32_t d_in, uint32_t t);

/* aur_outer_accum without any allocation: the same arithmetic (same launch
 * plan and kernels, so the same result bit for bit), with the split-K
 * partial tiles in a fixed scratch array the library holds on each device
 * (2^24 floats = 64 MiB, a file-scope __device__ array, present from library
 * load until the process ends) instead of the context's grow-on-demand
 * workspace.  It calls no hipMalloc / hipFree and never synchronises.
 * No counterpart in the reference: it is for callers that cannot allocate —
 * work captured into a HIP graph, tight serving loops, harnesses that
 * forbid allocation.  Shapes whose partial tiles need more than the scratch
 * return AUR_ELIMIT before anything is launched.  Every call on one device
 * shares that device's array; nothing in it needs clearing (each call writes
 * the partial tiles it reads back), but calls that overlap on one device —
 * from two contexts' streams, say — race on it. */
int aur_outer_accum_noalloc(aur_ctx* ctx, const float* x, const float* d_y, float* dest,
                            uint32_t d_out, uint32_t d_in, uint32_t t);

/* General strided form used by the model orchestrator (no reference
 * counterpart as one call: it is the union of the three kernels above with
 * explicit leading dimensions).
 *   a_kcontig != 0 : A(m,k) = a[m*lda + k]   else A(m,k) = a[k*lda + m]
 *   b_kcontig != 0 : B(k,n) = b[n*ldb + k]   else B(k,n) = b[k*ldb + n]
 *   C(m,n) = c[m*ldc + n];  accumulate != 0 → C += A·B  else C = A·B.
 * AUR_EINVAL when lda < (a_kcontig ? k : m), ldb < (b_kcontig ? k : n) or
 * ldc < n; AUR_ELIMIT for an extent above 2^31 - 1. */
int aur_gemm_ex(aur_ctx* ctx, int a_kcontig, int b_kcontig,
                const float* a, uint32_t lda, const float* b, uint32_t ldb,
                float* c, uint32_t ldc, uint32_t m, uint32_t n, uint32_t k,
                int accumulate);

/* ---- causal multi-head attention ----------------------------------------- */

/* Forward for a batch of `b` sequences: q,k,v,out are [b*t, n_head*d_head]
 * (head h at column offset h*d_head, the reference's per-sequence layout
 * with a leading batch axis); scale = 1/sqrt(d_head), causal mask j > i.
 * `lse` [b, n_head, t] receives each row's log-sum-exp of the scaled scores;
 * it takes the slot of the reference's `probs` [n_head,t,t], which no caller
 * reads back (it is only the forward→backward hand-off).
 * Replaces CausalMhaForwardKernel::dispatch_into(ctx, enc, q, k, v, out,
 * probs, t, n_head, d_head) (src/gpu/attention.rs:400-443).
 * Limits: any d_head from 1 to 64 (AUR_ELIMIT above, as the reference's
 * one-thread-per-column backward, src/gpu/attention.rs:266-331); multiples
 * of 8 run in place and need q/k/v/out 16-byte aligned, any other d_head
 * runs on zero-padded copies of the heads in the context's workspace
 * (allocated on first need, so not while the stream is being captured);
 * any t >= 1. */
int aur_mha_fwd(aur_ctx* ctx, const float* q, const float* k, const float* v,
                float* out, float* lse,
                uint32_t b, uint32_t t, uint32_t n_head, uint32_t d_head);

/* Backward: dq, dk, dv are ACCUMULATED (+=), the caller zeroes them first
 * (attention.rs:575-578).  Deterministic: every output element has exactly
 * one writer, three passes (row dot D = Σ dO⊙O; dK/dV over query tiles,
 * which also stores the dS tiles of the causal lower triangle; dQ = dS·K
 * over those tiles).  `ws` is a caller-owned workspace of at least
 * aur_mha_bwd_ws_bytes(b, t, n_head) bytes, which never exceeds the
 * reference's d_scores_scratch of n_head·t·t floats per sequence, and the
 * call writes no more of it than that: D [b,n_head,t] and the dS tiles,
 * ≈ b·n_head·t²/2 floats.  For short or ragged t, where the tiles need more
 * than b·n_head·t² floats, they go to the context's own workspace instead
 * (allocated on first need; AUR_EINVAL while the stream is being captured).
 * Replaces CausalMhaBackwardKernel::dispatch_into(ctx, enc, q, k, v, probs,
 * d_out, dq, dk, dv, d_scores_scratch, t, n_head, d_head)
 * (src/gpu/attention.rs:580-685). */
size_t aur_mha_bwd_ws_bytes(uint32_t b, uint32_t t, uint32_t n_head);
int aur_mha_bwd(aur_ctx* ctx, const float* q, const float* k, const float* v,
                const float* out, const float* lse, const float* d_out,
                float* dq, float* dk, float* dv, float* ws,
                uint32_t b, uint32_t t, uint32_t n_head, uint32_t d_head);

/* Strided forms (row strides in floats) used by the orchestrator to read
 * q/k/v straight out of a fused [rows, 3*d] QKV projection. */
int aur_mha_fwd_ex(aur_ctx* ctx, const float* q, const float* k, const float* v,
                   uint32_t ld_qkv, float* out, uint32_t ld_out, float* lse,
                   uint32_t b, uint32_t t, uint32_t n_head, uint32_t d_head);
int aur_mha_bwd_ex(aur_ctx* ctx, const float* q, const float* k, const float* v,
                   uint32_t ld_qkv, const float* out, const float* d_out,
                   uint32_t ld_out, const float* lse, float* dq, float* dk,
                   float* dv, uint32_t ld_dqkv, float* ws,
                   uint32_t b, uint32_t t, uint32_t n_head, uint32_t d_head);

/* ---- KV-cache decode attention --------------------------------------------- */

/* One new query per head against history rows [0, t_total):
 * q_new [n_head*d_head], k_history/v_history [max_len, n_head*d_head],
 * out [n_head*d_head].  `scratch` is caller-owned, at least
 * aur_mha_kv_ws_bytes(1, n_head, max_len) bytes, which never exceeds the
 * reference's n_head·max_len floats (src/gpu/transformer.rs:2432): 68-float
 * records per 128 keys where a full history's records fit in that, else 0
 * bytes (the scratch-free one-block-per-head kernel runs).  Any d_head >= 1
 * (the reference stride-loops over the head's columns, src/gpu/kv_cache.rs:
 * 339-348): multiples of 8 up to 64 take the bandwidth-shaped kernels, any
 * other d_head a generic one that keeps the scores of up to 16384 keys in
 * LDS (AUR_ELIMIT beyond).
 * Replaces MhaKvCacheKernel::dispatch_into(ctx, enc, q_new, k_history,
 * v_history, out, scratch, t_total, n_head, d_head, max_len)
 * (src/gpu/kv_cache.rs:421-465). */
size_t aur_mha_kv_ws_bytes(uint32_t b, uint32_t n_head, uint32_t max_len);
int aur_mha_kv_step(aur_ctx* ctx, const float* q_new, const float* k_history,
                    const float* v_history, float* out, float* scratch,
                    uint32_t t_total, uint32_t n_head, uint32_t d_head,
                    uint32_t max_len);

/* Batched form for `b` sequences decoded together: q_new/out [b, d],
 * k_history/v_history [b, max_len, d], per-sequence lengths in the DEVICE
 * array t_total[b] (1 <= t_total[i] <= max_len, max over i given as
 * t_max on the host).  No reference counterpart as one call: the reference
 * decodes one sequence per call (src/gpu/transformer.rs:2410). */
int aur_mha_kv_step_batched(aur_ctx* ctx, const float* q_new,
                            const float* k_history, const float* v_history,
                            float* out, float* scratch, const int32_t* t_total,
                            uint32_t t_max, uint32_t b, uint32_t n_head,
                            uint32_t d_head, uint32_t max_len);

/* ---- model: DecoderTransformerGpu / KvCacheGpu ----------------------------
 * The caller of the hot path (src/gpu/transformer.rs:32-116, 949-2640),
 * running B sequences through every GEMM together (M = B·T rows).  The
 * pre-LN GPT of the reference with optional features off: tied head, learned
 * positions, LayerNorm eps 1e-5, tanh-GELU FFN. */
typedef struct aur_model aur_model;
typedef struct aur_kv_cache aur_kv_cache;
typedef struct {
  uint32_t vocab, d_model, n_layer, n_head, d_ff, seq_len_max;
} aur_model_config; /* TransformerConfig, src/transformer/model.rs:24-127 */

/* DecoderTransformerGpu::from_cpu (transformer.rs:949) without the upload:
 * allocates parameters (zero), gradients, AdamW moments and the activation
 * arena for max_batch × seq_len_max rows.  Parameters are then written
 * through aur_model_tensor pointers.  Limits: d_model a multiple of n_head
 * with d_head = d_model / n_head up to 64 (AUR_ELIMIT above; d_head not a
 * multiple of 8 trains on zero-padded head copies in the context's workspace
 * and decodes through the generic KV kernel); vocab, d_model and d_ff
 * multiples of 4. */
int aur_model_create(aur_ctx* ctx, const aur_model_config* cfg, uint32_t max_batch, aur_model** out);
int aur_model_destroy(aur_model* m);
/* Device pointer + length of a parameter (grad = 0) or its gradient
 * (grad = 1): "w_tok", "w_pos", "lnf_g", "lnf_b", and per layer "ln1_g",
 * "ln1_b", "w_q", "w_k", "w_v" (rows of "w_qkv" = [w_q; w_k; w_v]), "w_o",
 * "ln2_g", "ln2_b", "w_fc", "w_proj"; "params" / "grads" are the flat
 * buffers.  Replaces the public field p: GpuParams (transformer.rs:86). */
int aur_model_tensor(aur_model* m, const char* name, int32_t layer, int32_t grad, float** ptr,
                     size_t* len);
/* zero_grad (transformer.rs:1242). */
int aur_model_zero_grad(aur_model* m);

/* ---- AURORA07 checkpoints (src/checkpoint.rs) ------------------------------
 * aur_checkpoint_peek reads the header of an AURORA05/06/07 file: the model
 * dimensions, the feature flags word (checkpoint.rs:70-79), epoch and step.
 * aur_model_load_checkpoint (checkpoint.rs:188-301 `load`, into an existing
 * model of the same dimensions): fills every parameter, zeroes the optimizer
 * moments and sets the optimizer step to the stored one; AUR_ELIMIT when the
 * file uses an optional feature this backend does not implement (any flag,
 * softcap, canon kernel, sink tokens), AUR_EINVAL on a bad magic or other
 * dimensions, AUR_EIO when the file cannot be read or ends early.
 * aur_model_save_checkpoint (checkpoint.rs:84-186 `save`): writes AURORA07
 * with every optional feature off. */
int aur_checkpoint_peek(const char* path, aur_model_config* cfg, uint32_t* flags, uint32_t* epoch,
                        uint64_t* step);
int aur_model_load_checkpoint(aur_model* m, const char* path, uint32_t* epoch, uint64_t* step);
int aur_model_save_checkpoint(aur_model* m, const char* path, uint32_t epoch, uint64_t step);
/* train_step_batch (transformer.rs:1571): forward + softmax-CE + backward for
 * b host sequences of length t (tokens/targets [b*t]); gradients accumulate
 * (+=, zero_grad first).  Each sequence's loss is its mean-over-t NLL
 * (model.rs:820-858); `reduction` says how the b gradients combine:
 *   AUR_BATCH_SUM  — summed, the reference GPU model's convention
 *                    (transformer.rs:1555-1559; its trainer then clips at
 *                    B × the threshold, examples/aurora_train.rs:1046-1051);
 *   AUR_BATCH_MEAN — averaged, the CPU trainer's grads.scale(1/B)
 *                    (examples/aurora_train.rs:840-846).
 * train_step (transformer.rs:1535) is the b = 1 case of either.
 * *loss_sum = Σ_b mean_t NLL_b (the reference's return value). */
#define AUR_BATCH_MEAN 0u
#define AUR_BATCH_SUM 1u
int aur_model_train_step_batch_ex(aur_model* m, const uint32_t* tokens, const uint32_t* targets,
                                  uint32_t b, uint32_t t, uint32_t reduction, float* loss_sum);
/* The AUR_BATCH_MEAN form of aur_model_train_step_batch_ex. */
int aur_model_train_step_batch(aur_model* m, const uint32_t* tokens, const uint32_t* targets,
                               uint32_t b, uint32_t t, float* loss_sum);
/* Forward only (encode_forward, transformer.rs:1347); logits [b*t, vocab]
 * copied to the host buffer `logits` when non-NULL. */
int aur_model_forward(aur_model* m, const uint32_t* tokens, uint32_t b, uint32_t t, float* logits);
/* eval_step_batch (transformer.rs:1734-1775; eval_step_per_token :1779-1811
 * is the b = 1 case, eval_step :1723 its sum): forward + softmax-CE at loss
 * scale 1, no backward, for b windows of length t (tokens/targets [b*t]);
 * nll[b*t] receives the per-token NLL in nats, window-major.  Parameters,
 * gradients and optimizer state are left untouched. */
int aur_model_eval_step_batch(aur_model* m, const uint32_t* tokens, const uint32_t* targets,
                              uint32_t b, uint32_t t, float* nll);
/* grad_norm (transformer.rs:1263): global L2 norm over all gradients. */
int aur_model_grad_norm(aur_model* m, float* norm);
/* clip_grads (model.rs:1011-1017): global L2 over all gradients, scaled in
 * place when above max_norm; *norm = the pre-clip norm.  With norm == NULL
 * the norm is not read back (no host synchronisation), like the reference's
 * want_norm = false (transformer.rs:2294); the same holds for the other
 * clipping entry points below. */
int aur_model_clip_grads(aur_model* m, float max_norm, float* norm);
/* step_adamw (model.rs:926-1009, transformer.rs:2008). */
int aur_model_step_adamw(aur_model* m, float lr, float beta1, float beta2, float eps,
                         float weight_decay);
/* step_muon_hybrid (model.rs:1023-1090, gpu/transformer.rs:2052-2291): the
 * reference trainer's default optimizer.  AdamW (lr, beta1, beta2, eps,
 * weight_decay; decay on w_tok only) on the embeddings and LayerNorm γ/β;
 * Muon (muon_lr, momentum, nesterov, muon_wd, ns_steps; optimizer.rs:
 * 94-305) on every w_q, w_k, w_v, w_o, w_fc, w_proj: momentum, Frobenius
 * bound, ns_steps quintic Newton–Schulz iterations on the GEMMs, scale
 * √(max/min).  Shares the AdamW step counter.  The Muon momentum buffers
 * are allocated (and zeroed) on the first call. */
int aur_model_step_muon_hybrid(aur_model* m, float muon_lr, float momentum, int32_t nesterov,
                               float muon_wd, uint32_t ns_steps, float lr, float beta1, float beta2,
                               float eps, float weight_decay);
/* clip_grads_adamw_subset (model.rs:1101-1107, gpu/transformer.rs:2294):
 * the L2 norm and the clip over the AdamW subset only (embeddings + LN). */
int aur_model_clip_grads_adamw_subset(aur_model* m, float max_norm, float* norm);
/* clip_grads + step_adamw fused (the clip factor is applied inside AdamW). */
int aur_model_clip_step_adamw(aur_model* m, float max_norm, float lr, float beta1, float beta2,
                              float eps, float weight_decay, float* norm);
/* snapshot_state / refresh_state / restore_state (transformer.rs:1152-1240):
 * the persistent state — parameters, both AdamW moments and the Muon
 * momentum (allocated with the model, like the reference's mu buffers, so
 * the size is fixed for the model's lifetime) — copied device-to-device into
 * / out of a caller-owned DEVICE buffer of `bytes` bytes (enqueued, no host
 * sync); `bytes` must equal aur_model_state_bytes, else AUR_EINVAL and
 * nothing is copied.  The optimizer step counter is returned / set
 * alongside. */
int aur_model_state_bytes(aur_model* m, size_t* bytes);
int aur_model_state_save(aur_model* m, void* dst, size_t bytes, uint64_t* step);
int aur_model_state_load(aur_model* m, const void* src, size_t bytes, uint64_t step);

/* KvCacheGpu::new (kv_cache.rs:42) for `batch` sequences decoded together,
 * max_len <= seq_len_max; reset zeroes it (kv_cache.rs:76).  A cache serves
 * only the model it was created from (prefill / generate_step with another
 * model return AUR_EINVAL).  Destroying the model detaches its caches: they
 * then accept only aur_kv_cache_destroy (and reset / len / history), and
 * decoding with them returns AUR_EINVAL. */
int aur_kv_cache_create(aur_model* m, uint32_t batch, uint32_t max_len, aur_kv_cache** out);
int aur_kv_cache_reset(aur_kv_cache* c);
int aur_kv_cache_destroy(aur_kv_cache* c);
int aur_kv_cache_len(aur_kv_cache* c, uint32_t* len);
/* Device K / V history of `layer`, each [batch, max_len, d_model]. */
int aur_kv_cache_history(aur_kv_cache* c, uint32_t layer, float** k, float** v);
/* prefill_kv (transformer.rs:2374; CPU KvCache::prefill kv_cache.rs:70):
 * full forward of b prompts of length t filling the cache; last-position
 * logits [b, vocab] to the host when non-NULL; the cache's next input
 * tokens become their argmax (the first greedy token). */
int aur_model_prefill_kv(aur_model* m, aur_kv_cache* c, const uint32_t* tokens, uint32_t b,
                         uint32_t t, float* last_logits);
/* generate_step_kv (transformer.rs:2410; CPU generate_step kv_cache.rs:97)
 * for all b sequences: `tokens` [b] from the host, or NULL to feed the
 * previous step's argmax (greedy, no host round trip).  Logits [b, vocab]
 * and the argmax tokens [b] are copied out when the pointers are non-NULL. */
int aur_model_generate_step(aur_model* m, aur_kv_cache* c, const uint32_t* tokens, float* logits,
                            uint32_t* next_tokens);
/* n_steps greedy generate_step calls; out_tokens [n_steps, b] or NULL. */
int aur_model_generate_greedy(aur_model* m, aur_kv_cache* c, uint32_t n_steps, uint32_t* out_tokens);

#ifdef __cplusplus
}
#endif
#endif /* AURORA_HIP_H */
