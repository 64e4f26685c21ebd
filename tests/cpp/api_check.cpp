// C++ API check of aurora_amd/csrc/aurora.hpp (the reference crate's kernel
// structs, DecoderTransformerGpu and KvCacheGpu, src/gpu/mod.rs:40-63), built
// with g++ against libaurora_hip.so.
//   api_check          no GPU expected: GpuContext construction must throw
//                      aurora::Error with aur_init's message (the reference's
//                      GpuContext::new() -> Err, context.rs:22).
//   api_check gpu      on a GPU: a GEMM-NT and an outer accumulate through the
//                      kernel structs against plain loops in double, attention
//                      forward + backward on a tiny shape against the same
//                      restated definition, and one model train step + a KV
//                      decode step (finite outputs, greedy token in range).
// Exit status 0 on success; the failing check is printed.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../aurora_amd/csrc/aurora.hpp"

using aurora::GpuBuffer;
using aurora::GpuContext;

namespace {

int fail(const char* what, double v) {
  std::printf("FAIL %s (%g)\n", what, v);
  return 1;
}

std::vector<float> uniform(size_t n, unsigned seed) {
  std::mt19937 g(seed);
  std::uniform_real_distribution<float> u(-1.f, 1.f);
  std::vector<float> v(n);
  for (auto& x : v) x = u(g);
  return v;
}

double rel(const std::vector<float>& a, const std::vector<double>& b) {
  double num = 0, den = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    num += (a[i] - b[i]) * (a[i] - b[i]);
    den += b[i] * b[i];
  }
  return std::sqrt(num / (den > 0 ? den : 1));
}

int gpu_checks() {
  GpuContext ctx(0);
  // y = x·Wᵀ (GemmTransposeBKernel) and dest += dYᵀ·X (OuterProductAccumKernel)
  const uint32_t m = 96, k = 64, n = 80;
  auto x = uniform(m * k, 1), w = uniform(n * k, 2), dy = uniform(m * n, 3), dest0 = uniform(n * k, 4);
  auto bx = GpuBuffer<float>::from_slice(ctx, x), bw = GpuBuffer<float>::from_slice(ctx, w);
  auto by = GpuBuffer<float>::zeros(ctx, m * n);
  aurora::GemmTransposeBKernel{}.dispatch_into(ctx, bx, bw, by, m, n, k);
  std::vector<double> want(m * n, 0.0);
  for (uint32_t i = 0; i < m; ++i)
    for (uint32_t j = 0; j < n; ++j)
      for (uint32_t c = 0; c < k; ++c) want[i * n + j] += (double)x[i * k + c] * w[j * k + c];
  if (double e = rel(by.download(), want); !(e < 1e-5)) return fail("GemmTransposeBKernel", e);
  auto bdy = GpuBuffer<float>::from_slice(ctx, dy), bdest = GpuBuffer<float>::from_slice(ctx, dest0);
  aurora::OuterProductAccumKernel{}.dispatch_into(ctx, bx, bdy, bdest, n, k, m);
  std::vector<double> acc(n * k);
  for (uint32_t o = 0; o < n; ++o)
    for (uint32_t i = 0; i < k; ++i) {
      double s = dest0[o * k + i];
      for (uint32_t t = 0; t < m; ++t) s += (double)dy[t * n + o] * x[t * k + i];
      acc[o * k + i] = s;
    }
  if (double e = rel(bdest.download(), acc); !(e < 1e-5)) return fail("OuterProductAccumKernel", e);
  // A buffer shorter than the dimensions name is refused before any launch.
  {
    auto short_c = GpuBuffer<float>::zeros(ctx, m * n - 1);
    bool refused = false;
    try {
      aurora::GemmTransposeBKernel{}.dispatch_into(ctx, bx, bw, short_c, m, n, k);
    } catch (const aurora::Error& e) {
      refused = e.code == AUR_EINVAL;
    }
    if (!refused) return fail("short output buffer accepted", 0);
  }

  // causal attention, t = 24, 2 heads of 16: O against the textbook definition
  const uint32_t t = 24, H = 2, dh = 16, d = H * dh;
  auto q = uniform(t * d, 5), kk = uniform(t * d, 6), v = uniform(t * d, 7);
  auto bq = GpuBuffer<float>::from_slice(ctx, q), bk = GpuBuffer<float>::from_slice(ctx, kk),
       bv = GpuBuffer<float>::from_slice(ctx, v);
  auto bo = GpuBuffer<float>::zeros(ctx, t * d), blse = GpuBuffer<float>::zeros(ctx, H * t);
  aurora::CausalMhaForwardKernel{}.dispatch_into(ctx, bq, bk, bv, bo, blse, t, H, dh);
  std::vector<double> o(t * d, 0.0);
  for (uint32_t h = 0; h < H; ++h)
    for (uint32_t i = 0; i < t; ++i) {
      std::vector<double> s(i + 1);
      double mx = -1e300, sum = 0;
      for (uint32_t j = 0; j <= i; ++j) {
        double a = 0;
        for (uint32_t c = 0; c < dh; ++c) a += (double)q[i * d + h * dh + c] * kk[j * d + h * dh + c];
        s[j] = a / std::sqrt((double)dh);
        mx = std::max(mx, s[j]);
      }
      for (uint32_t j = 0; j <= i; ++j) sum += (s[j] = std::exp(s[j] - mx));
      for (uint32_t j = 0; j <= i; ++j)
        for (uint32_t c = 0; c < dh; ++c) o[i * d + h * dh + c] += s[j] / sum * v[j * d + h * dh + c];
    }
  if (double e = rel(bo.download(), o); !(e < 1e-5)) return fail("CausalMhaForwardKernel", e);
  auto bdo = GpuBuffer<float>::from_slice(ctx, uniform(t * d, 8));
  auto dq = GpuBuffer<float>::zeros(ctx, t * d), dk = GpuBuffer<float>::zeros(ctx, t * d),
       dv = GpuBuffer<float>::zeros(ctx, t * d);
  GpuBuffer<float> ws(ctx, aurora::CausalMhaBackwardKernel::workspace_len(t, H));
  aurora::CausalMhaBackwardKernel{}.dispatch_into(ctx, bq, bk, bv, bo, blse, bdo, dq, dk, dv, ws, t, H, dh);
  for (float g : dq.download())
    if (!std::isfinite(g)) return fail("CausalMhaBackwardKernel dq not finite", g);

  // model: one train step (sum over the batch), clip + AdamW, then KV decode
  aurora::TransformerConfig cfg{64, 32, 1, 2, 64, 16};
  aurora::DecoderTransformerGpu model(ctx.raw(), cfg, 2);
  size_t np = 0;
  float* params = model.tensor("params", -1, false, &np);
  auto p = uniform(np, 9);
  for (auto& z : p) z *= 0.05f;
  if (aur_h2d(ctx.raw(), params, p.data(), np * 4)) return fail("upload params", 0);
  std::vector<uint32_t> tok(2 * 16), tgt(2 * 16);
  for (size_t i = 0; i < tok.size(); ++i) {
    tok[i] = (uint32_t)(i * 7 % 64);
    tgt[i] = (uint32_t)(i * 5 % 64);
  }
  model.zero_grad();
  const float loss = model.train_step_batch(tok.data(), tgt.data(), 2, 16, aurora::BatchReduction::Sum);
  if (!(std::fabs(loss / 2 - std::log(64.0)) < 0.5)) return fail("train_step_batch loss", loss);
  const float gn = model.grad_norm();
  const float cn = model.clip_and_step_adamw(1.0f, aurora::AdamWConfig{});
  if (!(gn > 0 && std::fabs(gn - cn) < 1e-5f * gn)) return fail("grad_norm vs clip norm", gn - cn);
  aurora::KvCacheGpu cache(model, 2, 16);
  std::vector<float> last(2 * 64);
  model.prefill_kv(cache, tok.data(), 2, 8, last.data());
  std::vector<float> logits(2 * 64);
  std::vector<uint32_t> next(2);
  model.generate_step_kv(cache, nullptr, logits.data(), next.data());
  if (cache.current_len != 9) return fail("KvCacheGpu current_len", cache.current_len);
  for (uint32_t b = 0; b < 2; ++b) {
    uint32_t best = 0;
    for (uint32_t c = 1; c < 64; ++c)
      if (logits[b * 64 + c] > logits[b * 64 + best]) best = c;
    if (next[b] != best) return fail("greedy token", next[b]);
  }
  std::printf("OK gpu: GEMM, outer accumulate, attention, train step (loss %.4f, norm %.4f), KV decode\n", loss, gn);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
  if (!gpu) {
    // Kernel structs are stateless values, as the reference's are after new().
    aurora::GemmKernel g1;
    aurora::GemmTransposeBKernel g2;
    aurora::OuterProductAccumKernel g3;
    aurora::CausalMhaForwardKernel a1;
    aurora::CausalMhaBackwardKernel a2;
    aurora::MhaKvCacheKernel a3;
    (void)g1, (void)g2, (void)g3, (void)a1, (void)a2, (void)a3;
    if (aurora::CausalMhaBackwardKernel::workspace_len(1024, 8, 16) * 4 != aur_mha_bwd_ws_bytes(16, 1024, 8))
      return fail("workspace_len", 0);
    try {
      GpuContext ctx(0);
      std::printf("a device is present: run with 'gpu'\n");
      return 0;
    } catch (const aurora::Error& e) {
      if (e.code == 0 || std::strlen(e.what()) == 0) return fail("aurora::Error without code/message", e.code);
      std::printf("OK no-gpu: GpuContext::new failed cleanly (code %d): %s\n", e.code, e.what());
      return 0;
    }
  }
  try {
    return gpu_checks();
  } catch (const aurora::Error& e) {
    std::printf("FAIL aurora::Error %d: %s\n", e.code, e.what());
    return 1;
  }
}
