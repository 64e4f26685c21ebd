"""Pins the CPU oracle (oracle/oracle.c + oracle/model.py) before it is trusted
as the checker of the GPU path.  CPU only.

Each oracle function is checked against something independent of its own
formula: PyTorch float64 library routines frozen in tests/golden/fixtures.npz
(layer norm, tanh-GELU, cross-entropy, causal SDPA, AdamW), numpy float64
matrix products, closed forms (AdamW's first step, embedding gather /
scatter), central-difference gradients of the whole model (the reference's
own check, tests/transformer_primitives.rs:21-93, EPS 1e-3, TOL 5e-2), and
the reference's invariants (KV decode == full forward, kv_cache.rs:64-138;
causal future independence, transformer_primitives.rs:179).

Parity status per oracle function — every one is pinned:
  dot, cpu_gemm, cpu_gemm_transpose_b, linear_forward/backward,
  outer_accum, tied_head_forward, lm_head_backward ......... numpy float64
  sdpa_forward/backward, mha_heads_* ...... torch SDPA fixture + float64
  layer_norm_*, gelu*, softmax_ce ................. torch fixtures
  adamw_apply, bias_correction ..... torch AdamW fixture + closed form
  embed_forward/backward ................................ closed form
  kv_attend ........................... last row of sdpa_forward
  model forward/backward ........ central differences + the above
  model assembly (block wiring, batch mean, clip + AdamW decay groups,
  AdamW-subset norm, Muon hybrid rows × cols) ..... torch float64 tiny GPT
                                 from primitives (tests/golden/model_fixture.npz)
  generate_step ...................... full forward (last row)
"""
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from oracle import model as OM

FX = np.load(Path(__file__).resolve().parent / "golden" / "fixtures.npz", allow_pickle=False)


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# ---------------------------------------------------------------- fixtures
def test_layer_norm_matches_torch():
    x, g, b, dy = FX["ln_x"], FX["ln_g"], FX["ln_b"], FX["ln_dy"]
    y, cache = O.layer_norm_forward(g, b, x.ravel(), 24)
    assert rel(y, FX["ln_y"]) < 1e-6
    dg, db = np.zeros(24, np.float32), np.zeros(24, np.float32)
    dx = O.layer_norm_backward(g, cache, dy.ravel(), dg, db, 24)
    assert rel(dx, FX["ln_dx"]) < 1e-5
    assert rel(dg, FX["ln_dg"]) < 1e-5 and rel(db, FX["ln_db"]) < 1e-5


def test_gelu_matches_torch():
    assert rel(O.gelu(FX["gelu_x"]), FX["gelu_y"]) < 1e-6
    assert rel(O.gelu_backward(FX["gelu_x"]), FX["gelu_dy"]) < 1e-6


def test_softmax_ce_matches_torch():
    total, d = O.softmax_ce(FX["ce_logits"].ravel(), FX["ce_tgt"], 33)
    t = FX["ce_tgt"].size
    assert abs(total / t - float(FX["ce_loss"])) < 1e-5
    assert rel(d, FX["ce_grad"]) < 1e-5


def test_sdpa_matches_torch():
    q, k, v, do = (FX[f"sdpa_{n}"] for n in ("q", "k", "v", "do"))
    out, probs = O.sdpa_forward(q.ravel(), k.ravel(), v.ravel(), 8, 8, causal=True)
    assert rel(out, FX["sdpa_o"]) < 1e-5
    P = probs.reshape(13, 13)
    assert np.allclose(P.sum(1), 1.0, atol=1e-6) and np.all(np.triu(P, 1) == 0)
    dq, dk, dv = O.sdpa_backward(q.ravel(), k.ravel(), v.ravel(), probs, do.ravel(), 8, 8)
    assert rel(dq, FX["sdpa_dq"]) < 1e-5
    assert rel(dk, FX["sdpa_dk"]) < 1e-5
    assert rel(dv, FX["sdpa_dv"]) < 1e-5


def test_adamw_matches_torch_two_steps():
    p0, p1 = FX["adam_p0"].astype(np.float32), FX["adam_p1"].astype(np.float32)
    s = {k: np.zeros_like(p) for k, p in (("a0", p0), ("b0", p0), ("a1", p1), ("b1", p1))}
    for step in (1, 2):
        bc1, bc2 = O.bias_correction(step, 0.9, 0.95)
        O.adamw_apply(p0, FX[f"adam_g0_s{step}"], s["a0"], s["b0"], 3e-4, 0.9, 0.95, 1e-8, 0.1, bc1, bc2, True)
        O.adamw_apply(p1, FX[f"adam_g1_s{step}"], s["a1"], s["b1"], 3e-4, 0.9, 0.95, 1e-8, 0.1, bc1, bc2,
                      False)
        np.testing.assert_allclose(p0, FX[f"adam_p0_s{step}"], rtol=0, atol=2e-7)
        np.testing.assert_allclose(p1, FX[f"adam_p1_s{step}"], rtol=0, atol=2e-7)


def test_adamw_first_step_closed_form():
    """At t = 1 with bias correction, m̂ = g and v̂ = g², so the update is
    lr·g/(|g| + eps) (+ lr·wd·θ on decayed groups)."""
    rng = np.random.default_rng(0)
    p = rng.standard_normal(50).astype(np.float32)
    g = rng.standard_normal(50).astype(np.float32)
    want = p - (3e-4 * g / (np.abs(g) + 1e-8) + 3e-4 * 0.1 * p)
    m1, m2 = np.zeros_like(p), np.zeros_like(p)
    bc1, bc2 = O.bias_correction(1, 0.9, 0.95)
    O.adamw_apply(p, g, m1, m2, 3e-4, 0.9, 0.95, 1e-8, 0.1, bc1, bc2, True)
    np.testing.assert_allclose(p, want, rtol=0, atol=1e-6)


# ------------------------------------------------------------------ GEMMs
@pytest.mark.parametrize("m,k,n", [(5, 7, 3), (16, 33, 9), (33, 64, 17)])
def test_gemm_oracles_match_float64(m, k, n):
    rng = np.random.default_rng(m * 100 + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert rel(O.cpu_gemm(a, b, m, k, n), ref) < 1e-6
    assert rel(O.cpu_gemm_transpose_b(a, np.ascontiguousarray(b.T), m, k, n), ref) < 1e-6
    # linear_forward: y = x·Wᵀ with W [d_out, d_in] = bᵀ
    w = np.ascontiguousarray(b.T)
    assert rel(O.linear_forward(w, a, k, n), ref) < 1e-6
    assert rel(O.tied_head_forward(a, w, n, k), ref) < 1e-6


def test_dot_is_eight_lane_fma():
    rng = np.random.default_rng(3)
    for n in (1, 7, 8, 9, 64, 100):
        a, b = rng.uniform(-1, 1, n).astype(np.float32), rng.uniform(-1, 1, n).astype(np.float32)
        assert abs(O.dot(a, b) - float(a.astype(np.float64) @ b.astype(np.float64))) < 1e-5


def test_linear_backward_matches_float64():
    rng = np.random.default_rng(5)
    t, d_in, d_out = 19, 12, 10
    w = rng.uniform(-1, 1, (d_out, d_in)).astype(np.float32)
    x = rng.uniform(-1, 1, (t, d_in)).astype(np.float32)
    dy = rng.uniform(-1, 1, (t, d_out)).astype(np.float32)
    dw0 = rng.uniform(-1, 1, (d_out, d_in)).astype(np.float32)
    dw = dw0.copy()
    dx = O.linear_backward(w, x, dy, dw, d_in, d_out)
    assert rel(dx, dy.astype(np.float64) @ w) < 1e-6
    assert rel(dw, dw0 + dy.T.astype(np.float64) @ x) < 1e-6
    # lm_head_backward is the same algebra with the head layout
    dh = np.zeros_like(dw0)
    dhead = O.lm_head_backward(x, w, dy, dh, d_out, d_in)
    assert rel(dhead, dy.astype(np.float64) @ w) < 1e-6 and rel(dh, dy.T.astype(np.float64) @ x) < 1e-6


def test_outer_accum_matches_float64():
    rng = np.random.default_rng(6)
    t, d_in, d_out = 23, 9, 14
    x = rng.uniform(-1, 1, (t, d_in)).astype(np.float32)
    dy = rng.uniform(-1, 1, (t, d_out)).astype(np.float32)
    dest0 = rng.uniform(-1, 1, (d_out, d_in)).astype(np.float32)
    dest = dest0.copy()
    O.outer_accum(x, dy, dest, d_out, d_in, t)
    assert rel(dest, dest0 + dy.T.astype(np.float64) @ x) < 1e-6


# -------------------------------------------------------------- attention
def test_mha_heads_match_float64_and_future_independence():
    from tests.attn_ref import causal_attention_f64, causal_attention_grad_f64

    rng = np.random.default_rng(8)
    t, H, dh = 17, 3, 8
    q, k, v, do = (rng.standard_normal((t, H * dh)).astype(np.float32) for _ in range(4))
    out, probs = O.mha_heads_forward(q, k, v, t, H, dh)
    o64, _ = causal_attention_f64(*(a.reshape(1, t, H, dh).astype(np.float64) for a in (q, k, v)))
    assert rel(out, o64) < 1e-5
    grads = O.mha_heads_backward(q, k, v, probs, do, t, H, dh)
    g64 = causal_attention_grad_f64(*(a.reshape(1, t, H, dh).astype(np.float64) for a in (q, k, v, do)))
    for g, w in zip(grads, g64):
        assert rel(g, w) < 1e-5
    k2 = k.copy()
    k2[9:] += 1.0
    out2, _ = O.mha_heads_forward(q, k2, v, t, H, dh)
    assert np.array_equal(out.reshape(t, -1)[:9], out2.reshape(t, -1)[:9])


def test_kv_attend_is_last_row_of_sdpa():
    rng = np.random.default_rng(9)
    t, H, dh = 11, 2, 8
    q, k, v = (rng.standard_normal((t, H * dh)).astype(np.float32) for _ in range(3))
    full, _ = O.mha_heads_forward(q, k, v, t, H, dh)
    for tt in (1, 5, 11):
        got = O.kv_attend(q[tt - 1], k, v, tt, H, dh)
        np.testing.assert_allclose(got, full.reshape(t, -1)[tt - 1], rtol=1e-5, atol=1e-6)


def test_embedding_closed_form():
    rng = np.random.default_rng(10)
    V, T, d = 7, 5, 4
    w_tok = rng.standard_normal((V, d)).astype(np.float32)
    w_pos = rng.standard_normal((T, d)).astype(np.float32)
    tok = np.array([3, 0, 3, 6, 3], np.uint32)
    out = O.embed_forward(w_tok, w_pos, tok, d).reshape(T, d)
    assert np.array_equal(out, w_tok[tok] + w_pos[:T])
    dy = rng.standard_normal((T, d)).astype(np.float32)
    gt, gp = np.zeros((V, d), np.float32), np.zeros((T, d), np.float32)
    O.embed_backward(tok, dy, gt, gp, d)
    want = np.zeros((V, d))
    np.add.at(want, tok, dy.astype(np.float64))
    assert rel(gt, want) < 1e-6 and np.array_equal(gp, dy)


# -------------------------------------------------------------- model level
TINY = OM.Config(vocab=16, d_model=16, n_layer=1, n_head=2, d_ff=32, seq_len_max=8)


def _loss(P, cfg, tok, tgt):
    logits, _ = OM.forward(P, cfg, tok)
    total, _ = O.softmax_ce(logits, tgt, cfg.vocab)
    return total / len(tok)


def test_model_gradient_matches_central_differences():
    """transformer_primitives.rs:21-93 style: EPS 1e-3, TOL 5e-2 relative."""
    cfg = TINY
    P = OM.init_params(cfg, 3)
    rng = np.random.default_rng(4)
    # larger weights than the 0.02 init so the gradients stand clear of fp32 noise
    for _, _, a in OM.tensors(P):
        a += rng.standard_normal(a.shape).astype(np.float32) * 0.3
    tok = rng.integers(0, cfg.vocab, 6).astype(np.uint32)
    tgt = rng.integers(0, cfg.vocab, 6).astype(np.uint32)
    G = OM.zeros_like(P)
    logits, cache = OM.forward(P, cfg, tok)
    OM.backward(P, cfg, cache, logits, tgt, G)
    eps = 1e-3
    checked = 0
    for (name, l, p), (_, _, g) in zip(OM.tensors(P), OM.tensors(G)):
        flat, gflat = p.reshape(-1), g.reshape(-1)
        idx = rng.choice(flat.size, size=min(4, flat.size), replace=False)
        if name == "w_pos":
            idx = np.array([0, 1 * cfg.d_model + 3, 5 * cfg.d_model + 1])  # rows that are used
        for i in idx:
            old = flat[i]
            flat[i] = old + eps
            lp = _loss(P, cfg, tok, tgt)
            flat[i] = old - eps
            lm = _loss(P, cfg, tok, tgt)
            flat[i] = old
            num = (lp - lm) / (2 * eps)
            ana = float(gflat[i])
            assert abs(num - ana) <= 5e-2 * max(abs(num), abs(ana)) + 3e-4, (name, l, i, num, ana)
            checked += 1
    assert checked > 40


def test_generate_step_equals_full_forward():
    """kv_cache.rs:64-138: prefill + generate_step logits == forward's last row."""
    cfg = OM.Config(vocab=32, d_model=32, n_layer=2, n_head=2, d_ff=64, seq_len_max=32)
    P = OM.init_params(cfg, 7)
    rng = np.random.default_rng(7)
    seq = rng.integers(0, cfg.vocab, 12).astype(np.uint32)
    kv = OM.KvCache(cfg)
    kv.prefill(P, seq[:6])
    for i in range(6, 12):
        step_logits = OM.generate_step(P, cfg, kv, int(seq[i]))
        full, _ = OM.forward(P, cfg, seq[:i + 1])
        np.testing.assert_allclose(step_logits, full.reshape(i + 1, -1)[-1], rtol=0, atol=5e-5)


def test_batch_grads_are_mean_of_sequences():
    """stability.rs:167-202 (additivity) with the CPU trainer's 1/B scale."""
    cfg = TINY
    P = OM.init_params(cfg, 11)
    rng = np.random.default_rng(11)
    tok = rng.integers(0, cfg.vocab, (2, 7)).astype(np.uint32)
    tgt = rng.integers(0, cfg.vocab, (2, 7)).astype(np.uint32)
    loss, G = OM.batch_grads(P, cfg, tok, tgt)
    singles = []
    for b in range(2):
        g = OM.zeros_like(P)
        lg, c = OM.forward(P, cfg, tok[b])
        OM.backward(P, cfg, c, lg, tgt[b], g)
        singles.append(g)
    for (_, _, gb), (_, _, g0), (_, _, g1) in zip(OM.tensors(G), OM.tensors(singles[0]),
                                                 OM.tensors(singles[1])):
        np.testing.assert_allclose(gb, (g0 + g1) / 2, rtol=0, atol=1e-6)


def test_batch_grads_threads_and_sum_mode():
    """The threaded oracle (sequences concurrently, summed in sequence order)
    is bit-identical to the serial one; the sum mode is the mean mode times B
    (the GPU model's convention, gpu/transformer.rs:1555-1559)."""
    cfg = TINY
    P = OM.init_params(cfg, 12)
    rng = np.random.default_rng(12)
    tok = rng.integers(0, cfg.vocab, (4, cfg.seq_len_max)).astype(np.uint32)
    tgt = rng.integers(0, cfg.vocab, (4, cfg.seq_len_max)).astype(np.uint32)
    l1, G1 = OM.batch_grads(P, cfg, tok, tgt)
    l4, G4 = OM.batch_grads(P, cfg, tok, tgt, threads=4)
    ls, Gs = OM.batch_grads(P, cfg, tok, tgt, threads=3, reduction="sum")
    assert l1 == l4 == ls
    for (_, _, a), (_, _, b), (_, _, s) in zip(OM.tensors(G1), OM.tensors(G4), OM.tensors(Gs)):
        assert np.array_equal(a, b)
        np.testing.assert_allclose(s, 4 * a.astype(np.float64), rtol=1e-6, atol=1e-9)


def test_embed_refuses_positions_past_the_table():
    """A sequence longer than w_pos has rows is an error (the reference indexes
    w_pos[pos] and panics), not an out-of-bounds read."""
    import oracle as O
    with pytest.raises(ValueError):
        O.embed_forward(np.zeros((5, 4), np.float32), np.zeros((3, 4), np.float32),
                        np.zeros(4, np.uint32), 4)


# ------------------------------------- model assembly vs the torch fixture
# tests/golden/model_fixture.npz holds a tiny pre-LN GPT written from torch
# primitives alone (tests/golden/make_fixtures.py), independent of oracle/:
# its forward wiring, autograd gradients, clip + AdamW with the reference's
# decay groups and the Muon hybrid step pin how oracle/model.py assembles the
# primitives that the tests above pin one by one.
MFX = np.load(Path(__file__).resolve().parent / "golden" / "model_fixture.npz", allow_pickle=False)
MCFG = OM.Config(*(int(v) for v in MFX["cfg"]))


def _fixture_tree(prefix):
    """A fixture's flat 'l{l}.key' arrays as the oracle's parameter dict."""
    P = {k: MFX[f"{prefix}.{k}"].astype(np.float32).copy() for k in ("w_tok", "w_pos", "lnf_g", "lnf_b")}
    P["layers"] = [{k: MFX[f"{prefix}.l{l}.{k}"].astype(np.float32).copy() for k in OM.LAYER_KEYS}
                   for l in range(MCFG.n_layer)]
    return P


def _pairs(A, prefix):
    for name, l, a in OM.tensors(A):
        key = name if l < 0 else f"l{l}.{name}"
        yield key, a, MFX[f"{prefix}.{key}"]


def test_model_forward_matches_torch_definition():
    """Logits and per-sequence mean NLL of the oracle's forward equal the
    torch model's (pre-LN blocks, LN2 on the post-attention residual, final
    LN, tied head)."""
    P = _fixture_tree("p")
    V = MCFG.vocab
    for b in range(MFX["tokens"].shape[0]):
        logits, _ = OM.forward(P, MCFG, MFX["tokens"][b])
        assert rel(logits, MFX["logits"][b]) < 2e-6, b
        total, _ = O.softmax_ce(logits, MFX["targets"][b], V)
        assert abs(total / MFX["targets"].shape[1] - MFX["seq_loss"][b]) < 2e-6 * MFX["seq_loss"][b]


def test_model_batch_grads_match_torch_autograd():
    P = _fixture_tree("p")
    loss, G = OM.batch_grads(P, MCFG, MFX["tokens"], MFX["targets"])
    assert abs(loss - MFX["seq_loss"].sum()) < 1e-5
    n = 0
    for key, g, want in _pairs(G, "g"):
        assert rel(g, want) < 2e-5, key
        n += 1
    assert n == 4 + 10 * MCFG.n_layer
    # rows of w_pos past t get no gradient
    assert not np.any(G["w_pos"][MFX["tokens"].shape[1]:])


def test_clip_and_adamw_match_torch_with_reference_decay_groups():
    """clip_grads (model.rs:1011-1017) at half the norm, then one step_adamw:
    w_tok, w_q/k/v/o, w_fc, w_proj decayed; w_pos and LayerNorm γ/β not."""
    P = _fixture_tree("p")
    G = _fixture_tree("g")
    n = OM.clip_grads(G, float(MFX["clip_max_norm"]))
    assert abs(n - float(MFX["grad_norm"])) < 1e-5 * n
    OM.step_adamw(P, G, OM.new_adam_state(P), lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.1)
    p0 = _fixture_tree("p")
    for (key, p, want), (_, _, start) in zip(_pairs(P, "adamw"), _pairs(p0, "p")):
        # compare the step itself: parameters move by ~lr, fp32 keeps ~1e-7·|θ|
        step, want_step = p.astype(np.float64) - start, want - start.astype(np.float64)
        assert np.max(np.abs(step - want_step)) < 2e-7 * max(1.0, np.max(np.abs(start))) + 1e-3 * 3e-4, key


def test_muon_hybrid_matches_torch_definition():
    """clip_grads_adamw_subset (model.rs:1101-1107; the norm over the subset
    of model.rs:518-560) and two step_muon_hybrid calls with the same
    gradients (AdamW on the subset, Muon with the reference's rows × cols
    on the block matrices) against the torch float64 restatement."""
    P = _fixture_tree("p")
    G = _fixture_tree("g")
    n = OM.clip_grads_adamw_subset(G, float(MFX["subset_max_norm"]))
    assert abs(n - float(MFX["subset_norm"])) < 1e-5 * n
    adam, muon = OM.new_adam_state(P), OM.new_muon_state(P)
    prev = _fixture_tree("p")
    for step in (1, 2):
        OM.step_muon_hybrid(P, G, adam, muon, MCFG)
        for (key, p, want), (_, _, before) in zip(_pairs(P, f"muon{step}"), _pairs(prev, "p" if step == 1 else
                                                                                  f"muon{step - 1}")):
            upd = p.astype(np.float64) - before.astype(np.float64)
            want_upd = want - before.astype(np.float64)
            # Muon moves a matrix by lr·√(max/min)·(orthogonalised update):
            # compare the update; AdamW entries move by ~lr
            assert rel(upd, want_upd) < 2e-4, (step, key)
        prev = OM.copy_params(P)
