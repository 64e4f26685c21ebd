// Launchers of the step-support kernels (step_ops.hip).  All enqueue on the
// context's stream and return 0 or an error code.
#pragma once

#include "common.hpp"

namespace aur {

// out[r] = w_tok[tok[r]] + w_pos[pos(r)], pos(r) = pos_dev ? pos_dev[r] : r % T;
// lens (optional): lens[r] = pos(r) + 1, the decode step's attention length.
int embed_forward(aur_ctx* ctx, const float* w_tok, const float* w_pos, const uint32_t* tok,
                  const int32_t* pos_dev, int T, float* out, int rows, int d, int32_t* lens = nullptr);
// g_w_tok[tok_ids[u]] += Σ dy[row_idx[row_off[u]..row_off[u+1])]; g_w_pos[t] += Σ_b dy[b*T+t].
int embed_backward(aur_ctx* ctx, const float* dy, int B, int T, int d, const uint32_t* tok_ids,
                   const int32_t* row_off, const int32_t* row_idx, int n_unique, float* g_w_tok,
                   float* g_w_pos);

int layer_norm_forward(aur_ctx* ctx, const float* x, const float* gamma, const float* beta, float* y,
                       float* mean, float* rstd, int rows, int d, float eps);
// x = R + Σ_{z<np} P[z] (P: [np][rows][d], summed in z order), x_out = x,
// y = LN(x).  d % 4 == 0, d <= 4096.
int layer_norm_forward_sum(aur_ctx* ctx, const float* R, const float* P, int np, float* x_out,
                           const float* gamma, const float* beta, float* y, int rows, int d, float eps);
size_t layer_norm_backward_ws_floats(int rows, int d);
// dx = LN'(dy) [+ dres]; dgamma/dbeta accumulated (fixed-order column sums in ws).
int layer_norm_backward(aur_ctx* ctx, const float* x, const float* mean, const float* rstd,
                        const float* gamma, const float* dy, const float* dres, float* dx,
                        float* dgamma, float* dbeta, float* ws, int rows, int d);

// In place: logits → (softmax − onehot)·scale; nll[r] per row.
int softmax_ce(aur_ctx* ctx, float* logits, const uint32_t* targets, float* nll, int rows, int V,
               float scale);

// stats[0] = ‖g‖₂ over n floats, stats[1] = clip factor for max_norm.
int grad_norm(aur_ctx* ctx, const float* g, size_t n, float max_norm, float* part, float* stats);
size_t grad_norm_ws_floats();
// The same over two ranges (g1[0, n1) and g2[0, n2)): the AdamW subset of a
// Muon step (embeddings + LayerNorm, model.rs:514-560).
int grad_norm2(aur_ctx* ctx, const float* g1, size_t n1, const float* g2, size_t n2, float max_norm,
               float* part, float* stats);
// stats[0] = ‖x‖_F, stats[1] = 1/(‖x‖_F + 1e-7).
int frob_inv(aur_ctx* ctx, const float* x, size_t n, float* part, float* stats);
// Muon pieces (optimizer.rs:147-305, gpu/muon.rs).
int muon_momentum(aur_ctx* ctx, const float* g, float* m, float* upd, size_t n, float beta, bool nesterov);
// out = a·I + b·A + c·A² for nb stacked m × m matrices (Newton–Schulz).
int ns_combine(aur_ctx* ctx, float* out, const float* A, const float* A2, float a, float b, float c, int m,
               int nb);
int transpose(aur_ctx* ctx, const float* src, float* dst, int rows, int cols);
int muon_apply(aur_ctx* ctx, float* p, const float* upd, size_t n, float lr_scale, float lr_wd);
int scale_by(aur_ctx* ctx, float* x, size_t n, const float* factor);
int adamw(aur_ctx* ctx, float* p, const float* g, float* m1, float* m2, size_t n, size_t n_decay,
          const float* clip, float lr, float b1, float b2, float eps, float wd, float bc1, float bc2);

// K/V rows of a fused qkv [rows, 3d] into the history [B, max_len, d].
int kv_store(aur_ctx* ctx, const float* qkv, int d, float* kh, float* vh, int max_len,
             const int32_t* pos_dev, int rows, int T);
// out[r] = first argmax of logits row r; pos[r] += 1 when pos is non-null.
int argmax_rows(aur_ctx* ctx, const float* logits, int rows, int V, uint32_t* out, int32_t* pos = nullptr);
// Decode input row: x = w_tok[tok] + w_pos[pos], lens = pos + 1, y = LN(x).
int embed_layer_norm(aur_ctx* ctx, const float* w_tok, const float* w_pos, const uint32_t* tok,
                     const int32_t* pos_dev, float* x_out, const float* gamma, const float* beta, float* y,
                     int32_t* lens, int rows, int d, float eps);
// dst[r] = src[(r*row_step + row_off) * ld_src .. + d]
int gather_rows(aur_ctx* ctx, const float* src, int ld_src, int row_step, int row_off, float* dst,
                int rows, int d);

// Floats of the attention backward's tiled workspace (D + the causal dS
// tiles) that mha_bwd_store's ws must hold (attention.hip).
size_t mha_bwd_tiled_ws_floats(int b, int t, int n_head);
// aur_mha_bwd_ex that STORES dq/dk/dv instead of accumulating (attention.hip).
int mha_bwd_store(aur_ctx* ctx, const float* q, const float* k, const float* v, int ld_qkv, const float* out,
                  const float* d_out, int ld_out, const float* lse, float* dq, float* dk, float* dv, int ld_dqkv,
                  float* ws, int b, int t, int n_head, int d_head);

// Batched KV decode attention with q rows of stride ld_q (kv_decode.hip).
// k_new/v_new (same stride as q): the row at position t_total-1 is taken from
// them and appended to the history by the kernel.  nparts > 1: q, k_new and
// v_new are each the sum of nparts (≤ 8) K-range partial rows part_stride
// floats apart (the QKV projection's partials), summed in order.
// Weights of the GEMMs that follow the decode attention, to be pulled into
// the L2 of the XCD whose blocks will read them while the attention streams
// the K/V history (which it loads non-temporally, past L2).  Matrix m is
// [rows[m], row_floats[m]] row-major; its consumer runs column blocks of
// group[m] weight rows, block x on XCD x % 8 (the consumer's gridDim.x is a
// multiple of 8 and workgroups go to the XCDs round-robin), so XCD j gets
// the row groups x ≡ j (mod 8).
struct L2Prefetch {
  int nmat = 0;
  const float* ptr[3] = {nullptr, nullptr, nullptr};
  int rows[3] = {0, 0, 0};
  int row_floats[3] = {0, 0, 0};
  int group[3] = {0, 0, 0};
  int blocks_per_xcd = 0;  // prefetch blocks per XCD appended to the launch
  float* sink = nullptr;   // 1 float, written only if the loaded values sum to a sentinel
};

int mha_kv_batched(aur_ctx* ctx, const float* q, int ld_q, const float* k_history,
                   const float* v_history, float* out, float* scratch, const int32_t* t_total, int t_max,
                   int b, int n_head, int d_head, int max_len, const float* k_new = nullptr,
                   const float* v_new = nullptr, int nparts = 1, size_t part_stride = 0,
                   const L2Prefetch* prefetch = nullptr);

}  // namespace aur
