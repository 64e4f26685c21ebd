"""Parity at the BASELINE sizes (configs 3 and 4), through the C ABI.

* Config-3 width against the CPU oracle: the C3 layer shapes (V 8192,
  d 1024, H 16, d_ff 4096) at M = B·T = 16 × 1024 rows — the 256×128 GEMM
  tile, the split-K weight-gradient accumulate at t = 16384, the
  row-resident softmax-CE at V = 8192 and the fused LayerNorm backward at
  d = 1024 — with one layer (the layer count changes no kernel), plus a
  ragged small case.  The oracle runs its sequences on a thread pool as the
  reference's rayon loop does (examples/aurora_train.rs:828-838).
* The full config-3 model (12 layers, B 16, T 1024, BASELINE init with the
  1/√(2L) residual scaling): directional derivatives of the loss, central
  differences (L(θ+εu) − L(θ−εu)) / 2ε against ⟨g, u⟩, along the gradient of
  single tensors and of all parameters — a size-independent check of the
  whole backward (the reference's numerical-gradient test,
  tests/transformer_primitives.rs:40-93, scaled up).
* Config 4 in full: 32 prompts of 512, all 256 greedy decode steps (KV to
  768): every step's logits against one full forward over the generated
  sequences, greedy tokens against that forward's argmax position by
  position (first divergence and near-ties reported), generate_greedy
  against the step-by-step tokens, and fresh prefills at steps 1, 128, 255
  (tests/kv_cache.rs:166-213, 283-329).
"""
import os
import time

import numpy as np
import pytest

from oracle import model as OM
from tests.parity import fro_rel

pytestmark = pytest.mark.gpu

C3 = OM.Config(vocab=8192, d_model=1024, n_layer=12, n_head=16, d_ff=4096, seq_len_max=1024)


def _threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _tokens(vocab, B, T, seed):
    rng = np.random.default_rng(seed)
    seq = rng.integers(0, vocab, (B, T + 1)).astype(np.uint32)
    return seq[:, :T].copy(), seq[:, 1:].copy()


def _model(ctx, cfg, max_batch, P):
    from aurora_amd.model import DecoderTransformerGpu

    m = DecoderTransformerGpu(ctx, cfg.vocab, cfg.d_model, cfg.n_layer, cfg.n_head, cfg.d_ff,
                              cfg.seq_len_max, max_batch)
    m.load_params(P)
    return m


@pytest.mark.parametrize("n_layer,B,T", [(1, 16, 1024), (2, 2, 64)])
def test_config3_width_grads_match_oracle(ctx, n_layer, B, T):
    cfg = OM.Config(vocab=8192, d_model=1024, n_layer=n_layer, n_head=16, d_ff=4096, seq_len_max=1024)
    P = OM.init_params(cfg, 2)
    tok, tgt = _tokens(cfg.vocab, B, T, 2)
    m = _model(ctx, cfg, B, P)
    m.zero_grad()
    loss_gpu = m.train_step_batch(tok, tgt)
    G_gpu = m.read_tensors(grad=True)
    m.destroy()
    t0 = time.time()
    loss_cpu, G = OM.batch_grads(P, cfg, tok, tgt, threads=_threads())
    print(f"[c3 width L{n_layer} B{B} T{T}] oracle {time.time() - t0:.1f} s on {_threads()} threads", flush=True)
    assert abs(loss_gpu - loss_cpu) < 1e-5 * abs(loss_cpu), (loss_gpu, loss_cpu)
    worst, where = 0.0, None
    for (name, l, g), (_, _, w) in zip(OM.tensors(G_gpu), OM.tensors(G)):
        e = fro_rel(g, w)
        if e > worst:
            worst, where = e, (name, l)
        assert e < 1e-3, (name, l, e)
    print(f"[c3 width L{n_layer} B{B} T{T}] loss gpu {loss_gpu:.6f} cpu {loss_cpu:.6f}; "
          f"worst grad rel err {worst:.2e} at {where}", flush=True)


def test_config3_full_model_directional_derivatives(ctx):
    P = OM.init_params(C3, 2)
    tok, tgt = _tokens(C3.vocab, 16, 1024, 2)
    m = _model(ctx, C3, 16, P)
    del P
    m.zero_grad()
    loss = m.train_step_batch(tok, tgt) / 16  # mean-mode grads: ∇ of this mean loss
    # logits at init have std ≈ 0.64, so E[NLL] ≈ ln V + σ²/2 ≈ 9.2
    assert abs(loss - np.log(C3.vocab)) < 0.5, loss
    g_all = m.get("grads")
    assert np.all(np.isfinite(g_all))
    # bitwise repeatable
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    assert np.array_equal(g_all, m.get("grads"))
    del g_all

    def mean_loss():
        return float(np.mean(m.eval_step_batch(tok, tgt).astype(np.float64)))

    assert abs(mean_loss() - loss) < 1e-6 * loss
    dirs = [("w_tok", -1), ("w_pos", -1), ("w_q", 0), ("w_k", 6), ("w_v", 11), ("w_o", 5), ("w_fc", 11),
            ("w_proj", 0), ("ln1_g", 3), ("ln2_b", 7), ("lnf_g", -1), ("params", -1)]
    worst = 0.0
    for name, layer in dirs:
        theta = m.get(name, layer)
        g = m.get(name, layer, grad=True).astype(np.float64)
        gn = float(np.linalg.norm(g))
        u = g / gn
        eps = 2e-3 / gn  # the loss moves by ~2e-3 each way
        lp = lm = None
        for sgn in (1.0, -1.0):
            m.set(name, (theta + sgn * eps * u).astype(np.float32), layer)
            if sgn > 0:
                lp = mean_loss()
            else:
                lm = mean_loss()
        m.set(name, theta, layer)
        fd = (lp - lm) / (2 * eps)
        rel = abs(fd - gn) / gn
        worst = max(worst, rel)
        print(f"[c3 ddir] {name}[{layer}]: |g| {gn:.6e} finite difference {fd:.6e} rel {rel:.2e}", flush=True)
        assert rel < 1e-2, (name, layer, gn, fd)
    assert abs(mean_loss() - loss) < 1e-6 * loss  # parameters restored
    print(f"[c3 ddir] worst relative error {worst:.2e}", flush=True)
    m.destroy()


def test_config4_all_256_decode_steps_match_full_forward(ctx):
    B, T0, steps = 32, 512, 256
    P = OM.init_params(C3, 2)
    m = _model(ctx, C3, B, P)
    del P
    prompts = np.random.default_rng(4).integers(0, C3.vocab, (B, T0)).astype(np.uint32)
    cache = m.kv_cache(B, T0 + steps)
    last = m.prefill_kv(cache, prompts)
    toks = [last.argmax(1).astype(np.uint32)]
    step_logits = np.empty((steps, B, C3.vocab), np.float32)
    for s in range(steps):
        lg, nxt = m.generate_step_kv(cache)  # feeds the previous argmax
        step_logits[s] = lg
        toks.append(nxt)
    assert cache.current_len == T0 + steps
    gen = np.stack(toks, axis=1)  # [B, 257]: t_0 from the prefill, t_{s+1} from step s
    # the bench's path: generate_greedy over a fresh cache gives the same tokens
    cache2 = m.kv_cache(B, T0 + steps)
    m.prefill_kv(cache2, prompts)
    greedy = m.generate_greedy(cache2, steps)
    assert np.array_equal(greedy.T, gen[:, 1:])
    cache2.destroy()
    # one full forward over the 768 fed tokens: position 511 + s predicts t_s
    seq = np.concatenate([prompts, gen[:, :steps]], axis=1)
    full = m.forward(seq).reshape(B, T0 + steps, C3.vocab)
    assert fro_rel(last, full[:, T0 - 1]) < 1e-4
    worst = 0.0
    for s in range(steps):
        e = fro_rel(step_logits[s], full[:, T0 + s])
        worst = max(worst, e)
        assert e < 1e-4, (s, e)
    preds = full[:, T0 - 1:].argmax(2)  # [B, 257]
    top2 = np.partition(full[:, T0 - 1:], -2, axis=2)[:, :, -2:]
    gap = top2[:, :, 1] - top2[:, :, 0]
    ties = gap <= 1e-3
    diff = preds != gen
    first = None
    if diff.any():
        b, p = np.argwhere(diff)[np.argsort(np.argwhere(diff)[:, 1])[0]]
        first = (int(p), int(b), float(gap[b, p]))
    print(f"[config4] {steps} steps x {B} sequences, KV 512..767: max rel |step - full| logits {worst:.2e}; "
          f"token mismatches {int(diff.sum())} (first: position {first}), near-ties (gap <= 1e-3) "
          f"{int(ties.sum())} of {ties.size}", flush=True)
    assert not (diff & ~ties).any(), first
    # fresh prefills over the grown sequences at steps 1, 128, 255
    ref = m.kv_cache(B, T0 + steps)
    for s in (1, 128, 255):
        lg = m.prefill_kv(ref, seq[:, :T0 + s + 1])
        assert fro_rel(step_logits[s], lg) < 1e-4, s
    ref.destroy()
    cache.destroy()
    m.destroy()
