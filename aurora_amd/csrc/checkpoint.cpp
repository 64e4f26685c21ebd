// AURORA07 checkpoint I/O for DecoderTransformerGpu (src/checkpoint.rs).
//
// Binary layout, little-endian (checkpoint.rs:9-49): 8-byte magic
// "AURORA05" / "AURORA06" / "AURORA07"; u32 vocab, d_model, n_layer, n_head,
// d_ff, seq_len_max, flags; f32 softcap; u32 canon_kernel (V6+); u32
// sink_tokens (V7+); u32 epoch; u64 step; then f32 tensors: w_tok, w_pos,
// [w_head, head_bias, sink when their features are on], per block ln1_γ,
// ln1_β, w_q, w_k, w_v, w_o, ln2_γ, ln2_β, w_fc, w_proj [+ feature tensors],
// final γ, final β.  Writes are always V7 (checkpoint.rs:91-186).
//
// This backend implements the base pre-LN GPT (no rope / rmsnorm / relu² /
// qk-norm / untied head / swiglu / layerscale / parallel block / diff-attn /
// head bias, softcap 0, no canon conv, no sink tokens); a checkpoint using
// any of them is refused with AUR_ELIMIT rather than silently misread.  As
// in checkpoint.rs:188-301, loading gives fresh optimizer moments and sets
// the step counter (AdamW bias correction) to the stored step.
#include <cstdio>
#include <cstring>
#include <vector>

#include "aurora.hpp"

namespace aurora {
namespace {

constexpr char kMagic5[8] = {'A', 'U', 'R', 'O', 'R', 'A', '0', '5'};
constexpr char kMagic6[8] = {'A', 'U', 'R', 'O', 'R', 'A', '0', '6'};
constexpr char kMagic7[8] = {'A', 'U', 'R', 'O', 'R', 'A', '0', '7'};

struct File {
  std::FILE* f = nullptr;
  File(const char* path, const char* mode) : f(std::fopen(path, mode)) {}
  ~File() {
    if (f) std::fclose(f);
  }
};

// Little-endian scalar I/O (x86-64 and gfx hosts are little-endian; the
// byte order is still spelled out so the format does not depend on it).
void put_u32(std::vector<unsigned char>& b, uint32_t v) {
  for (int i = 0; i < 4; ++i) b.push_back((unsigned char)(v >> (8 * i)));
}
void put_u64(std::vector<unsigned char>& b, uint64_t v) {
  for (int i = 0; i < 8; ++i) b.push_back((unsigned char)(v >> (8 * i)));
}
uint32_t get_u32(const unsigned char* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
uint64_t get_u64(const unsigned char* p) { return (uint64_t)get_u32(p) | (uint64_t)get_u32(p + 4) << 32; }

void read_exact(std::FILE* f, void* dst, size_t n, const char* what) {
  if (std::fread(dst, 1, n, f) != n)
    throw Error(std::string("checkpoint: file ends inside ") + what, AUR_EIO);
}

}  // namespace

CheckpointHeader read_checkpoint_header(const char* path) {
  if (!path) throw Error("checkpoint: null path", AUR_EINVAL);
  File file(path, "rb");
  if (!file.f) throw Error(std::string("checkpoint: cannot open ") + path, AUR_EIO);
  return read_checkpoint_header(file.f);
}

CheckpointHeader read_checkpoint_header(std::FILE* f) {
  unsigned char magic[8];
  read_exact(f, magic, 8, "the magic");
  CheckpointHeader h{};
  if (!std::memcmp(magic, kMagic5, 8))
    h.version = 5;
  else if (!std::memcmp(magic, kMagic6, 8))
    h.version = 6;
  else if (!std::memcmp(magic, kMagic7, 8))
    h.version = 7;
  else
    throw Error("checkpoint: bad magic, expected AURORA05, AURORA06 or AURORA07", AUR_EINVAL);
  unsigned char b[4 * 8];
  read_exact(f, b, 4 * 7 + 4, "the header");  // 6 dims + flags + softcap
  h.cfg.vocab = get_u32(b);
  h.cfg.d_model = get_u32(b + 4);
  h.cfg.n_layer = get_u32(b + 8);
  h.cfg.n_head = get_u32(b + 12);
  h.cfg.d_ff = get_u32(b + 16);
  h.cfg.seq_len_max = get_u32(b + 20);
  h.flags = get_u32(b + 24);
  const uint32_t sc = get_u32(b + 28);
  std::memcpy(&h.softcap, &sc, 4);
  if (h.version >= 6) {
    read_exact(f, b, 4, "the header");
    h.canon_kernel = get_u32(b);
  }
  if (h.version >= 7) {
    read_exact(f, b, 4, "the header");
    h.sink_tokens = get_u32(b);
  }
  read_exact(f, b, 12, "the header");
  h.epoch = get_u32(b);
  h.step = get_u64(b + 4);
  return h;
}

void DecoderTransformerGpu::save_checkpoint(const char* path, uint32_t epoch, uint64_t step_out) const {
  if (!path) throw Error("checkpoint: null path", AUR_EINVAL);
  std::vector<unsigned char> head(kMagic7, kMagic7 + 8);
  put_u32(head, cfg_.vocab);
  put_u32(head, cfg_.d_model);
  put_u32(head, cfg_.n_layer);
  put_u32(head, cfg_.n_head);
  put_u32(head, cfg_.d_ff);
  put_u32(head, cfg_.seq_len_max);
  put_u32(head, 0);  // flags: every optional feature off
  put_u32(head, 0);  // softcap 0.0f
  put_u32(head, 0);  // canon_kernel
  put_u32(head, 0);  // sink_tokens
  put_u32(head, epoch);
  put_u64(head, step_out);
  std::vector<float> host(n_params_);
  check(ctx_, aur_d2h(ctx_, host.data(), params_, n_params_ * sizeof(float)), "download params");
  File file(path, "wb");
  if (!file.f) throw Error(std::string("checkpoint: cannot create ") + path, AUR_EIO);
  auto put = [&](const void* p, size_t bytes) {
    if (std::fwrite(p, 1, bytes, file.f) != bytes) throw Error("checkpoint: write failed", AUR_EIO);
  };
  put(head.data(), head.size());
  auto put_tensor = [&](const char* name, int layer) {
    size_t n = 0;
    const float* dev = tensor(name, layer, false, &n);
    put(host.data() + (dev - params_), n * sizeof(float));
  };
  put_tensor("w_tok", 0);
  put_tensor("w_pos", 0);
  for (int l = 0; l < (int)cfg_.n_layer; ++l)
    for (const char* nm : {"ln1_g", "ln1_b", "w_q", "w_k", "w_v", "w_o", "ln2_g", "ln2_b", "w_fc", "w_proj"})
      put_tensor(nm, l);
  put_tensor("lnf_g", 0);
  put_tensor("lnf_b", 0);
  if (std::fflush(file.f) != 0) throw Error("checkpoint: write failed", AUR_EIO);
}

CheckpointHeader DecoderTransformerGpu::load_checkpoint(const char* path) {
  if (!path) throw Error("checkpoint: null path", AUR_EINVAL);
  File file(path, "rb");
  if (!file.f) throw Error(std::string("checkpoint: cannot open ") + path, AUR_EIO);
  const CheckpointHeader h = read_checkpoint_header(file.f);
  if (h.flags != 0 || h.softcap != 0.0f || h.canon_kernel != 0 || h.sink_tokens != 0)
    throw Error("checkpoint: uses features this backend does not implement (flags 0x" +
                    std::to_string(h.flags) + ", softcap, canon or sink tokens)",
                AUR_ELIMIT);
  const TransformerConfig& c = h.cfg;
  if (c.vocab != cfg_.vocab || c.d_model != cfg_.d_model || c.n_layer != cfg_.n_layer ||
      c.n_head != cfg_.n_head || c.d_ff != cfg_.d_ff || c.seq_len_max != cfg_.seq_len_max)
    throw Error("checkpoint: model dimensions differ from this model's", AUR_EINVAL);
  std::vector<float> host(n_params_);
  auto get_tensor = [&](const char* name, int layer) {
    size_t n = 0;
    const float* dev = tensor(name, layer, false, &n);
    read_exact(file.f, host.data() + (dev - params_), n * sizeof(float), name);
  };
  get_tensor("w_tok", 0);
  get_tensor("w_pos", 0);
  for (int l = 0; l < (int)cfg_.n_layer; ++l)
    for (const char* nm : {"ln1_g", "ln1_b", "w_q", "w_k", "w_v", "w_o", "ln2_g", "ln2_b", "w_fc", "w_proj"})
      get_tensor(nm, l);
  get_tensor("lnf_g", 0);
  get_tensor("lnf_b", 0);
  check(ctx_, aur_h2d(ctx_, params_, host.data(), n_params_ * sizeof(float)), "upload params");
  reset_optimizer_state();
  step = h.step;
  return h;
}

}  // namespace aurora
