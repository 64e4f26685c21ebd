"""Muon hybrid optimizer (src/optimizer.rs:94-305, model.rs:1023-1107,
src/gpu/muon.rs, gpu/transformer.rs:2052-2291).

CPU: the oracle's newton_schulz5 (oracle.c, restating optimizer.rs:147-252)
is pinned by what the mathematics fixes rather than by a second copy of
its loops: the quintic drives the singular values of a random matrix into
the Jordan band, it is equivariant under orthogonal maps (NS(Q·G) =
Q·NS(G)) and under transposition (the rows > cols path), and it is
invariant to a positive scale (the Frobenius bound).  muon_apply is then
checked against its closed form on a fresh momentum buffer, and the subset
clip against a float64 norm.  GPU: the model's clip + step_muon_hybrid
against the CPU oracle on BASELINE config 0, over two steps (momentum).
"""
import numpy as np
import pytest

import oracle as O
from oracle import model as OM
from tests.parity import fro_rel

C0 = OM.Config(vocab=256, d_model=128, n_layer=2, n_head=4, d_ff=512, seq_len_max=64)


def _ns(g, rows, cols, it=5):
    x = np.ascontiguousarray(g, np.float32).copy()
    O.newton_schulz5(x, rows, cols, it)
    return x


@pytest.mark.parametrize("rows,cols", [(64, 64), (48, 96), (96, 48)])
def test_ns5_is_the_scalar_quintic_on_singular_values(rows, cols):
    """X·Xᵀ-polynomial iterations act on each singular value alone:
    NS(G) = U·φ⁵(Σ / (‖G‖_F + 1e-7))·Vᵀ with φ(x) = 3.4445x − 4.7750x³ +
    2.0315x⁵ (optimizer.rs:145-146), evaluated here in float64 from the SVD —
    a formulation independent of the oracle's matrix loops."""
    g = np.random.default_rng(rows + cols).standard_normal((rows, cols)).astype(np.float32)
    u, sv, vt = np.linalg.svd(g.astype(np.float64), full_matrices=False)
    x = sv / (np.sqrt(np.sum(g.astype(np.float64) ** 2)) + 1e-7)
    for _ in range(5):
        x = 3.4445 * x - 4.7750 * x ** 3 + 2.0315 * x ** 5
    want = (u * x) @ vt
    assert fro_rel(_ns(g, rows, cols), want) < 2e-5


@pytest.mark.parametrize("rows,cols", [(64, 64), (48, 96), (96, 48)])
def test_ns_converges_into_the_quintic_band(rows, cols):
    """Iterated long enough, every singular value sits in the quintic's
    attracting band [0.68, 1.135] — orthogonalisation up to that band."""
    g = np.random.default_rng(rows * cols).standard_normal((rows, cols)).astype(np.float32)
    sv = np.linalg.svd(_ns(g, rows, cols, it=12).astype(np.float64), compute_uv=False)
    assert sv.min() > 0.67 and sv.max() < 1.14, (sv.min(), sv.max())


def test_ns5_orthogonal_equivariance_and_transpose():
    rng = np.random.default_rng(3)
    g = rng.standard_normal((32, 80)).astype(np.float32)
    q, _ = np.linalg.qr(rng.standard_normal((32, 32)))
    q = q.astype(np.float32)
    lhs = _ns(q @ g, 32, 80)
    rhs = q @ _ns(g, 32, 80)
    assert fro_rel(lhs, rhs) < 1e-4
    # rows > cols goes through the physical transpose: NS(Gᵀ) = NS(G)ᵀ
    t = _ns(np.ascontiguousarray(g.T), 80, 32)
    assert fro_rel(t, _ns(g, 32, 80).T) < 1e-5


def test_ns5_scale_invariance_and_zero():
    g = np.random.default_rng(4).standard_normal((40, 40)).astype(np.float32)
    assert fro_rel(_ns(3.5 * g, 40, 40), _ns(g, 40, 40)) < 1e-5
    z = np.zeros((8, 8), np.float32)
    np.testing.assert_array_equal(_ns(z, 8, 8), z)  # ‖g‖² ≤ 1e-30: left as is


def test_muon_apply_closed_form_fresh_momentum():
    """Fresh momentum, Nesterov: update = g + β·g, whose NS5 equals NS5(g)
    (scale invariance), so p ← p − lr·√(max/min)·NS5(g) − lr·wd·p."""
    rng = np.random.default_rng(5)
    rows, cols = 32, 128
    p = rng.standard_normal((rows, cols)).astype(np.float32)
    g = rng.standard_normal((rows, cols)).astype(np.float32)
    mom = np.zeros_like(p)
    p1 = p.copy()
    O.muon_apply(p1, g, mom, rows, cols, lr=0.02, momentum=0.95, nesterov=True, wd=0.1)
    want = p - 0.02 * np.sqrt(128 / 32) * _ns(g, rows, cols) - 0.02 * 0.1 * p
    assert fro_rel(p1 - p, want - p) < 1e-5
    np.testing.assert_allclose(mom, g, rtol=0, atol=0)  # m = 0.95·0 + g


def test_clip_subset_norm_matches_float64():
    P = OM.init_params(C0, 0)
    G = OM.zeros_like(P)
    rng = np.random.default_rng(6)
    for _, _, a in OM.tensors(G):
        a[...] = rng.standard_normal(a.shape, dtype=np.float32)
    subset = list(OM._adamw_subset(G))
    n64 = np.sqrt(sum(np.sum(np.asarray(a, np.float64) ** 2) for _, _, a in subset))
    w_q = G["layers"][0]["w_q"].copy()
    n = OM.clip_grads_adamw_subset(G, 1.0)
    assert abs(n - n64) < 1e-4 * n64
    n_after = np.sqrt(sum(np.sum(np.asarray(a, np.float64) ** 2) for _, _, a in OM._adamw_subset(G)))
    assert abs(n_after - 1.0) < 1e-5
    np.testing.assert_array_equal(G["layers"][0]["w_q"], w_q)  # matrices untouched


@pytest.mark.gpu
def test_gpu_muon_hybrid_matches_cpu(ctx):
    from aurora_amd.model import DecoderTransformerGpu

    cfg = C0
    P = OM.init_params(cfg, 0)
    rng = np.random.default_rng(0)
    seq = rng.integers(0, cfg.vocab, (8, 65)).astype(np.uint32)
    tok, tgt = seq[:, :64].copy(), seq[:, 1:].copy()
    m = DecoderTransformerGpu(ctx, cfg.vocab, cfg.d_model, cfg.n_layer, cfg.n_head, cfg.d_ff,
                              cfg.seq_len_max, 8)
    m.load_params(P)
    adam, muon = OM.new_adam_state(P), OM.new_muon_state(P)
    kw = dict(muon_lr=0.02, momentum=0.95, nesterov=True, muon_wd=0.01, ns_steps=5, lr=3e-4, wd=0.1)
    for step in range(2):
        P_before = OM.copy_params(P)
        m.zero_grad()
        m.train_step_batch(tok, tgt)
        n_gpu = m.clip_grads_adamw_subset(1.0)
        m.step_muon_hybrid(muon_lr=0.02, momentum=0.95, nesterov=True, muon_wd=0.01, ns_steps=5, lr=3e-4,
                           weight_decay=0.1)
        _, G = OM.batch_grads(P, cfg, tok, tgt)
        n_cpu = OM.clip_grads_adamw_subset(G, 1.0)
        OM.step_muon_hybrid(P, G, adam, muon, cfg, **kw)
        assert abs(n_gpu - n_cpu) < 1e-3 * n_cpu, (step, n_gpu, n_cpu)
        got = m.read_tensors(grad=False)
        worst = 0.0
        for (name, l, a), (_, _, b), (_, _, b0) in zip(OM.tensors(got), OM.tensors(P), OM.tensors(P_before)):
            # the step itself (p_new − p_old) to 1e-3, the parameters to 1e-5
            e = fro_rel(a - b0.ravel(), b.ravel() - b0.ravel())
            worst = max(worst, e)
            assert e < 1e-3, (step, name, l, e)
            assert fro_rel(a, b) < 1e-5, (step, name, l)
        print(f"[muon] step {step}: subset norm gpu {n_gpu:.6f} cpu {n_cpu:.6f}, worst update err {worst:.2e}")
        # the GPU keeps its own parameters; re-sync so step 2 starts from the same point
        m.load_params(P)
    m.destroy()
