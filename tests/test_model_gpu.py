"""GPU parity of the model level: DecoderTransformerGpu train step at
M = B·T and the batched KV-cache decode, through the C ABI.

Mirrors tests/gpu_parity.rs:569-1148 (loss |Δ| < 5e-2, grads < 5e-2,
train_step_loss_matches_cpu_baseline 5e-3, batch == Σ sequential) and
tests/kv_cache.rs (GPU KV vs CPU KV 5e-2 :232-279, greedy identity
:166-213 / :283-329, t_total > 64 stride loops :346-386), with the CPU
oracle (oracle.model) as the reference CPU path.
"""
import numpy as np
import pytest

from oracle import model as OM
from tests.parity import fro_rel

pytestmark = pytest.mark.gpu

# V256 d128 L2 H4 d_ff512 T64 B8, seed 0.
C0 = OM.Config(vocab=256, d_model=128, n_layer=2, n_head=4, d_ff=512, seq_len_max=64)


def _gpu_model(ctx, cfg, max_batch, P):
    from aurora_amd.model import DecoderTransformerGpu

    m = DecoderTransformerGpu(ctx, cfg.vocab, cfg.d_model, cfg.n_layer, cfg.n_head, cfg.d_ff,
                              cfg.seq_len_max, max_batch)
    m.load_params(P)
    return m


def _tokens(cfg, B, T, seed):
    rng = np.random.default_rng(seed)
    seq = rng.integers(0, cfg.vocab, (B, T + 1)).astype(np.uint32)
    return seq[:, :T].copy(), seq[:, 1:].copy()


def _compare_tree(got, want, tol, what):
    worst = 0.0
    for (name, l, g), (_, _, w) in zip(OM.tensors(got), OM.tensors(want)):
        e = fro_rel(g, w)
        worst = max(worst, e)
        assert e < tol, (what, name, l, e)
    return worst


@pytest.mark.parametrize("vocab", [1024, 2048])
def test_train_step_row_resident_ce_matches_cpu(ctx, vocab):
    """Vocabularies that are multiples of 1024 take the row-resident softmax-CE
    kernel (the C3 head, V = 8192, does too): loss and every gradient against
    the CPU restatement, including the tied embedding that the CE gradient
    feeds."""
    cfg = OM.Config(vocab=vocab, d_model=64, n_layer=1, n_head=2, d_ff=128, seq_len_max=32)
    P = OM.init_params(cfg, 5)
    tok, tgt = _tokens(cfg, 4, 32, 5)
    m = _gpu_model(ctx, cfg, 4, P)
    m.zero_grad()
    loss_gpu = m.train_step_batch(tok, tgt)
    loss_cpu, G = OM.batch_grads(P, cfg, tok, tgt)
    assert abs(loss_gpu - loss_cpu) < 1e-4 * abs(loss_cpu), (loss_gpu, loss_cpu)
    _compare_tree(m.read_tensors(grad=True), G, 1e-3, "grad")
    m.destroy()


def test_config0_train_step_matches_cpu(ctx):
    """One forward + backward + clip(1.0) + AdamW(lr 3e-4, wd 0.1) step."""
    cfg = C0
    P = OM.init_params(cfg, 0)
    tok, tgt = _tokens(cfg, 8, 64, 0)
    m = _gpu_model(ctx, cfg, 8, P)
    m.zero_grad()
    loss_gpu = m.train_step_batch(tok, tgt)
    G_gpu = m.read_tensors(grad=True)

    loss_cpu, G = OM.batch_grads(P, cfg, tok, tgt)
    assert abs(loss_gpu - loss_cpu) < 5e-3 * 8, (loss_gpu, loss_cpu)  # Σ over 8 sequence means
    worst_g = _compare_tree(G_gpu, G, 1e-3, "grad")

    # The reference's l2_norm is one sequential fp32 sum over ~0.5 M squares
    # (model.rs:442-500), the GPU's a fixed two-level tree: compare both with
    # the float64 norm of the same gradients, and with each other.
    n64_gpu = float(np.sqrt(sum(np.sum(np.asarray(g, np.float64) ** 2) for _, _, g in OM.tensors(G_gpu))))
    n64_cpu = float(np.sqrt(sum(np.sum(np.asarray(g, np.float64) ** 2) for _, _, g in OM.tensors(G))))
    norm_gpu = m.clip_grads(1.0)
    m.step_adamw(lr=3e-4, weight_decay=0.1)
    norm_cpu = OM.clip_grads(G, 1.0)
    st = OM.new_adam_state(P)
    OM.step_adamw(P, G, st, lr=3e-4, wd=0.1)
    print(f"[config0] norm gpu {norm_gpu:.7f} (f64 of gpu grads {n64_gpu:.7f}) "
          f"cpu {norm_cpu:.7f} (f64 of cpu grads {n64_cpu:.7f})")
    assert abs(norm_gpu - n64_gpu) < 1e-5 * n64_gpu
    assert abs(n64_gpu - n64_cpu) < 1e-4 * n64_cpu
    assert abs(norm_gpu - norm_cpu) < 1e-3 * norm_cpu, (norm_gpu, norm_cpu)
    worst_p = _compare_tree(m.read_tensors(grad=False), P, 1e-5, "param")
    print(f"[config0] loss gpu {loss_gpu:.6f} cpu {loss_cpu:.6f} |grad err| <= {worst_g:.2e} "
          f"norm {norm_gpu:.5f}/{norm_cpu:.5f} |param err| <= {worst_p:.2e}")
    m.destroy()


@pytest.mark.parametrize("d,B,T", [(256, 4, 256), (512, 3, 200), (1024, 2, 100), (2048, 2, 100)])
def test_train_step_wide_rows_matches_cpu(ctx, d, B, T):
    """d_model 256 / 512 / 1024 / 2048 over B·T = 1024 / 600 / 200 / 200
    rows: the row-resident float4 LayerNorm forward and the fused LayerNorm
    backward (dx with the γ/β chunk partials and the residual gradient loaded
    with x and dy; 600 and 200 rows leave a partial last chunk of 32 rows)
    against the oracle.  d = 1024 is the config-3 width; d = 2048 is the
    largest row the fused kernel holds."""
    cfg = OM.Config(vocab=128, d_model=d, n_layer=1, n_head=d // 64, d_ff=2 * d, seq_len_max=256)
    P = OM.init_params(cfg, 5)
    tok, tgt = _tokens(cfg, B, T, 5)
    m = _gpu_model(ctx, cfg, B, P)
    m.zero_grad()
    loss_gpu = m.train_step_batch(tok, tgt)
    loss_cpu, G = OM.batch_grads(P, cfg, tok, tgt)
    assert abs(loss_gpu - loss_cpu) < 5e-3 * B, (loss_gpu, loss_cpu)
    worst = _compare_tree(m.read_tensors(grad=True), G, 1e-3, "grad")
    print(f"[d{d} rows {B * T}] loss gpu {loss_gpu:.6f} cpu {loss_cpu:.6f} |grad err| <= {worst:.2e}")
    m.destroy()


@pytest.mark.parametrize("dh", [24, 40, 48, 56, 12, 20, 5])
def test_train_step_head_widths_match_cpu(ctx, dh):
    """d_head values that are multiples of 8 but not of 16, and ones that
    are not multiples of 8 (zero-padded heads), as the reference takes any
    d_head ≤ 64: one train step over 2 × 70 rows against the oracle, every
    gradient."""
    H = 4
    cfg = OM.Config(vocab=128, d_model=H * dh, n_layer=1, n_head=H, d_ff=2 * H * dh, seq_len_max=80)
    P = OM.init_params(cfg, 7)
    tok, tgt = _tokens(cfg, 2, 70, 7)
    m = _gpu_model(ctx, cfg, 2, P)
    m.zero_grad()
    loss_gpu = m.train_step_batch(tok, tgt)
    loss_cpu, G = OM.batch_grads(P, cfg, tok, tgt)
    assert abs(loss_gpu - loss_cpu) < 1e-4 * abs(loss_cpu), (loss_gpu, loss_cpu)
    worst = _compare_tree(m.read_tensors(grad=True), G, 1e-3, "grad")
    print(f"[d_head {dh}] loss gpu {loss_gpu:.6f} cpu {loss_cpu:.6f} |grad err| <= {worst:.2e}")
    m.destroy()


def test_fused_layernorm_backward_equals_unfused(ctx, monkeypatch):
    """d_model 1024 over 2 × 100 rows (seven 32-row chunks, the last one
    partial): the fused LayerNorm backward gives the gradients of the
    separate dx / γ-β partial kernels (AUR_LN_UNFUSED); dx is computed
    identically, dγ / dβ differ only in summation order."""
    cfg = OM.Config(vocab=64, d_model=1024, n_layer=1, n_head=16, d_ff=1024, seq_len_max=128)
    P = OM.init_params(cfg, 9)
    tok, tgt = _tokens(cfg, 2, 100, 9)
    grads = []
    for unfused in (False, True):
        if unfused:
            monkeypatch.setenv("AUR_LN_UNFUSED", "1")
        m = _gpu_model(ctx, cfg, 2, P)
        m.zero_grad()
        m.train_step_batch(tok, tgt)
        grads.append(m.read_tensors(grad=True))
        m.destroy()
    monkeypatch.delenv("AUR_LN_UNFUSED")
    for (name, l, a), (_, _, b) in zip(OM.tensors(grads[0]), OM.tensors(grads[1])):
        a, b = np.asarray(a), np.asarray(b)
        scale = max(1e-6, float(np.abs(b).max()))
        assert float(np.abs(a - b).max()) <= 1e-5 * scale, (name, l)


def test_sum_reduction_matches_reference_gpu_convention(ctx):
    """The reference GPU model's train_step_batch SUMS per-sequence gradients
    (src/gpu/transformer.rs:1555-1559) and its trainer clips at B × the
    threshold (examples/aurora_train.rs:1046-1051): the sum mode equals the
    oracle's summed grads, equals B × the mean mode, and clip(B·c) after it
    reports B × the norm of clip(c) after the mean mode and leaves B × its
    clipped gradients."""
    cfg = C0
    B = 8
    P = OM.init_params(cfg, 4)
    tok, tgt = _tokens(cfg, B, 64, 4)
    m = _gpu_model(ctx, cfg, B, P)
    m.zero_grad()
    loss_sum = m.train_step_batch(tok, tgt, reduction="sum")
    g_sum = m.get("grads")
    loss_cpu, G = OM.batch_grads(P, cfg, tok, tgt, reduction="sum")
    assert abs(loss_sum - loss_cpu) < 5e-3 * B, (loss_sum, loss_cpu)
    _compare_tree(m.read_tensors(grad=True), G, 1e-3, "sum grad")
    m.zero_grad()
    loss_mean = m.train_step_batch(tok, tgt, reduction="mean")
    g_mean = m.get("grads")
    assert loss_mean == loss_sum  # the returned loss is Σ_b mean_t NLL either way
    assert fro_rel(g_sum, B * g_mean.astype(np.float64)) < 1e-6
    # clip(B·c) after sum == B × clip(c) after mean
    c = 0.05
    m.zero_grad()
    m.train_step_batch(tok, tgt, reduction="sum")
    n_sum = m.clip_grads(B * c)
    gc_sum = m.get("grads")
    m.zero_grad()
    m.train_step_batch(tok, tgt, reduction="mean")
    n_mean = m.clip_grads(c)
    gc_mean = m.get("grads")
    assert n_mean > c  # the clip was active
    assert abs(n_sum - B * n_mean) < 1e-5 * n_sum, (n_sum, n_mean)
    assert fro_rel(gc_sum, B * gc_mean.astype(np.float64)) < 1e-6
    m.destroy()


def test_grad_norm_snapshot_and_optional_norm(ctx):
    """grad_norm (transformer.rs:1263) is the pre-clip norm and leaves the
    gradients alone; clip without a norm pointer clips the same way with no
    read-back; snapshot / restore (transformer.rs:1207-1240) bring back
    parameters, moments and the step counter bit for bit."""
    cfg = C0
    P = OM.init_params(cfg, 6)
    tok, tgt = _tokens(cfg, 4, 64, 6)
    m = _gpu_model(ctx, cfg, 4, P)
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    g0 = m.get("grads")
    n = m.grad_norm()
    assert np.array_equal(m.get("grads"), g0)
    assert abs(n - float(np.linalg.norm(g0.astype(np.float64)))) < 1e-5 * n
    assert np.isnan(m.clip_grads(0.5 * n, want_norm=False))
    assert fro_rel(m.get("grads"), g0 * np.float32(0.5)) < 1e-6
    m.step_adamw(lr=3e-4)
    snap = m.snapshot_state()
    assert snap.step == 1
    before = m.get("params")
    st_before = snap.download()
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    m.step_adamw(lr=3e-4)
    assert not np.array_equal(m.get("params"), before)
    m.restore_state(snap)
    assert np.array_equal(m.get("params"), before)
    again = m.snapshot_state()
    assert again.step == 1 and np.array_equal(again.download(), st_before)
    m.destroy()


def test_state_snapshot_size_fixed_across_muon(ctx):
    """The persistent state has one size for the model's lifetime: a snapshot
    taken before the first Muon step (whose momentum the reference keeps in
    its mu buffers from the start) still fits after it, round-trips the
    momentum, and a buffer of any other size is refused before any copy."""
    from aurora_amd._lib import AuroraError
    from aurora_amd.gpu import GpuBuffer
    cfg = C0
    P = OM.init_params(cfg, 7)
    tok, tgt = _tokens(cfg, 2, 64, 7)
    m = _gpu_model(ctx, cfg, 2, P)
    n0 = m.state_bytes()
    snap = m.snapshot_state()
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    m.step_muon_hybrid()
    assert m.state_bytes() == n0
    m.refresh_state(snap)
    after_one = snap.download()
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    m.step_muon_hybrid()
    assert not np.array_equal(m.snapshot_state().download(), after_one)
    m.restore_state(snap)
    assert np.array_equal(m.snapshot_state().download(), after_one)
    short = GpuBuffer.empty(ctx, n0 // 4 - 1)
    for bad in (lambda: m.refresh_state(short), lambda: m.restore_state(short)):
        short.step = 0
        with pytest.raises(AuroraError):
            bad()
    assert np.array_equal(m.snapshot_state().download(), after_one)
    m.destroy()


def test_kv_cache_belongs_to_its_model(ctx):
    """A cache's captured decode step holds its model's weight pointers: a
    second model may not use it, and once its model is destroyed the cache
    refuses decoding but can still be reset and destroyed."""
    from aurora_amd._lib import AuroraError

    cfg = OM.Config(vocab=64, d_model=64, n_layer=1, n_head=2, d_ff=128, seq_len_max=32)
    P = OM.init_params(cfg, 3)
    a, b = _gpu_model(ctx, cfg, 2, P), _gpu_model(ctx, cfg, 2, P)
    cache = a.kv_cache(2, 32)
    prompts = np.arange(16, dtype=np.uint32).reshape(2, 8)
    a.prefill_kv(cache, prompts)
    a.generate_step_kv(cache)
    with pytest.raises(AuroraError) as e:
        b.prefill_kv(cache, prompts)
    assert e.value.code == 10001
    with pytest.raises(AuroraError):
        b.generate_step_kv(cache)
    a.destroy()
    with pytest.raises(AuroraError) as e:
        b.generate_step_kv(cache)
    assert e.value.code == 10001
    cache.reset()
    assert cache.current_len == 0
    cache.destroy()
    b.destroy()


def test_fused_clip_adamw_equals_separate(ctx):
    cfg = C0
    P = OM.init_params(cfg, 1)
    tok, tgt = _tokens(cfg, 4, 64, 1)
    outs = []
    for fused in (False, True):
        m = _gpu_model(ctx, cfg, 4, P)
        m.zero_grad()
        m.train_step_batch(tok, tgt)
        if fused:
            m.clip_step_adamw(0.05, lr=3e-4, weight_decay=0.1)
        else:
            m.clip_grads(0.05)
            m.step_adamw(lr=3e-4, weight_decay=0.1)
        outs.append(m.get("params"))
        m.destroy()
    np.testing.assert_allclose(outs[0], outs[1], rtol=0, atol=1e-7)


def test_train_step_deterministic_and_batch_additive(ctx):
    cfg = C0
    P = OM.init_params(cfg, 2)
    tok, tgt = _tokens(cfg, 4, 64, 2)
    m = _gpu_model(ctx, cfg, 4, P)
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    g1 = m.get("grads")
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    g2 = m.get("grads")
    assert np.array_equal(g1, g2)  # bitwise run to run (no atomics anywhere)
    # batch of 4 == mean of two batches of 2 (stability.rs:167 additivity)
    m.zero_grad()
    m.train_step_batch(tok[:2], tgt[:2])
    ga = m.get("grads")
    m.zero_grad()
    m.train_step_batch(tok[2:], tgt[2:])
    gb = m.get("grads")
    assert fro_rel(g1, (ga + gb) / 2) < 1e-5
    m.destroy()


def test_ragged_seq_lengths_forward_matches_cpu(ctx):
    cfg = OM.Config(vocab=64, d_model=64, n_layer=2, n_head=4, d_ff=128, seq_len_max=100)
    P = OM.init_params(cfg, 5)
    m = _gpu_model(ctx, cfg, 3, P)
    for T in (1, 17, 65, 100):
        tok, _ = _tokens(cfg, 3, T, T)
        got = m.forward(tok)
        for b in range(3):
            want, _ = OM.forward(P, cfg, tok[b])
            assert fro_rel(got[b * T:(b + 1) * T], want) < 1e-4, (T, b)
    m.destroy()


# ------------------------------------------------------------------ decode
def test_kv_decode_matches_cpu_generate_step(ctx):
    """kv_cache.rs:232-279 at d_head 32, prompts 70 > 64 (stride loops)."""
    cfg = OM.Config(vocab=96, d_model=128, n_layer=2, n_head=4, d_ff=256, seq_len_max=96)
    P = OM.init_params(cfg, 9)
    B, T0, steps = 3, 70, 10
    rng = np.random.default_rng(9)
    prompts = rng.integers(0, cfg.vocab, (B, T0)).astype(np.uint32)
    feed = rng.integers(0, cfg.vocab, (steps, B)).astype(np.uint32)
    m = _gpu_model(ctx, cfg, B, P)
    cache = m.kv_cache(B, cfg.seq_len_max)
    last = m.prefill_kv(cache, prompts)
    cpu = [OM.KvCache(cfg) for _ in range(B)]
    for b in range(B):
        full = cpu[b].prefill(P, prompts[b])
        assert fro_rel(last[b], full.reshape(T0, -1)[-1]) < 1e-4
    for s in range(steps):
        logits, _ = m.generate_step_kv(cache, feed[s])
        for b in range(B):
            want = OM.generate_step(P, cfg, cpu[b], int(feed[s, b]))
            assert fro_rel(logits[b], want) < 1e-4, (s, b)
    assert cache.current_len == T0 + steps
    # the cached K/V rows equal the CPU cache's
    k0, v0 = cache.history(0)
    assert fro_rel(k0[1, :T0 + steps], cpu[1].k[0].reshape(T0 + steps, -1)) < 1e-4
    cache.destroy()
    m.destroy()


def test_kv_decode_above_64_sequences_matches_cpu(ctx):
    """More than 64 sequences: the decode step runs eagerly (no captured
    graph) with the tiled GEMMs and their residual epilogues instead of the
    decode K-range kernels; every sequence against the oracle."""
    cfg = OM.Config(vocab=64, d_model=64, n_layer=2, n_head=4, d_ff=128, seq_len_max=32)
    P = OM.init_params(cfg, 23)
    B, T0, steps = 72, 10, 3
    rng = np.random.default_rng(23)
    prompts = rng.integers(0, cfg.vocab, (B, T0)).astype(np.uint32)
    feed = rng.integers(0, cfg.vocab, (steps, B)).astype(np.uint32)
    m = _gpu_model(ctx, cfg, B, P)
    cache = m.kv_cache(B, cfg.seq_len_max)
    last = m.prefill_kv(cache, prompts)
    cpu = [OM.KvCache(cfg) for _ in range(B)]
    for b in range(B):
        full = cpu[b].prefill(P, prompts[b])
        assert fro_rel(last[b], full.reshape(T0, -1)[-1]) < 1e-4, b
    for s in range(steps):
        logits, nxt = m.generate_step_kv(cache, feed[s])
        for b in range(B):
            want = OM.generate_step(P, cfg, cpu[b], int(feed[s, b]))
            assert fro_rel(logits[b], want) < 1e-4, (s, b)
        assert np.array_equal(nxt, logits.argmax(1)), s
    assert cache.current_len == T0 + steps
    cache.destroy()
    m.destroy()


@pytest.mark.parametrize("d,H,F", [(384, 6, 1536), (768, 12, 3072), (640, 10, 2560), (384, 8, 1536),
                                   (96, 4, 192), (48, 4, 96), (80, 4, 160)])
def test_kv_decode_widths_match_cpu(ctx, d, H, F):
    """Decode at the reference's TransformerConfig::nano width (d 384, H 6,
    d_ff 1536; src/transformer/model.rs:87-96) and at d 768 / 640: K = 384,
    768, 1536, 2560, 3072 give split counts whose K ranges must all be
    non-empty (the W_o / W_proj partial products); d 384 with 8 heads and
    d 96 with 4 give d_head 48 and 24; d 48 and 80 with 4 heads give d_head
    12 and 20 (the new K/V rows appended by their own launch, the generic KV
    kernel, prefill through the padded attention)."""
    cfg = OM.Config(vocab=96, d_model=d, n_layer=2, n_head=H, d_ff=F, seq_len_max=48)
    P = OM.init_params(cfg, 17)
    B, T0, steps = 2, 20, 4
    rng = np.random.default_rng(17)
    prompts = rng.integers(0, cfg.vocab, (B, T0)).astype(np.uint32)
    feed = rng.integers(0, cfg.vocab, (steps, B)).astype(np.uint32)
    m = _gpu_model(ctx, cfg, B, P)
    cache = m.kv_cache(B, cfg.seq_len_max)
    last = m.prefill_kv(cache, prompts)
    cpu = [OM.KvCache(cfg) for _ in range(B)]
    for b in range(B):
        full = cpu[b].prefill(P, prompts[b])
        assert fro_rel(last[b], full.reshape(T0, -1)[-1]) < 1e-4
    for s in range(steps):
        logits, _ = m.generate_step_kv(cache, feed[s])
        for b in range(B):
            want = OM.generate_step(P, cfg, cpu[b], int(feed[s, b]))
            assert fro_rel(logits[b], want) < 1e-4, (d, s, b)
    cache.destroy()
    m.destroy()


def test_greedy_kv_decode_token_identical_to_full_forward(ctx):
    """kv_cache.rs:166-213 / :283-329: greedy tokens from the KV path equal the
    greedy tokens of a full forward over the growing sequence."""
    cfg = OM.Config(vocab=128, d_model=128, n_layer=2, n_head=2, d_ff=256, seq_len_max=64)
    P = OM.init_params(cfg, 13)
    B, T0, steps = 4, 20, 24
    rng = np.random.default_rng(13)
    prompts = rng.integers(0, cfg.vocab, (B, T0)).astype(np.uint32)
    m = _gpu_model(ctx, cfg, B, P)
    cache = m.kv_cache(B, cfg.seq_len_max)
    last = m.prefill_kv(cache, prompts)
    first = last.argmax(1).astype(np.uint32)
    toks = m.generate_greedy(cache, steps)  # toks[s] = argmax after feeding step s's token
    kv_seq = np.concatenate([prompts, first[:, None], toks.T], axis=1)  # T0 + 1 + steps
    # full-forward greedy on the same growing sequences (one batch forward per step)
    seq = np.concatenate([prompts, first[:, None]], axis=1)
    for s in range(steps):
        logits = m.forward(seq).reshape(B, seq.shape[1], -1)[:, -1]
        nxt = logits.argmax(1).astype(np.uint32)
        order = np.sort(logits, axis=1)
        gap = order[:, -1] - order[:, -2]
        assert np.array_equal(nxt, kv_seq[:, T0 + 1 + s]), (s, nxt, kv_seq[:, T0 + 1 + s], gap)
        seq = np.concatenate([seq, nxt[:, None]], axis=1)
    # and against the CPU oracle's greedy decode for one sequence
    kv = OM.KvCache(cfg)
    lg = kv.prefill(P, prompts[0])
    tok = OM.argmax(lg.reshape(T0, -1)[-1])
    cpu_seq = [tok]
    for _ in range(steps):
        lg = OM.generate_step(P, cfg, kv, tok)
        tok = OM.argmax(lg)
        cpu_seq.append(tok)
    assert cpu_seq == list(kv_seq[0, T0:]), (cpu_seq, kv_seq[0, T0:])
    cache.destroy()
    m.destroy()


def test_decode_l2_prefetch_leaves_results_unchanged(ctx, monkeypatch):
    """AUR_DEC_PREFETCH (read when the decode step is captured) appends
    blocks to the KV attention that pull the following GEMMs' weights into
    L2; they only load, so every logit of every step is bit-identical."""
    cfg = OM.Config(vocab=256, d_model=512, n_layer=2, n_head=16, d_ff=1024, seq_len_max=64)
    P = OM.init_params(cfg, 17)
    B = 32  # B·H = 512 pairs: the one-block-per-(sequence, head) kernel
    prompts = np.random.default_rng(17).integers(0, cfg.vocab, (B, 24)).astype(np.uint32)
    m = _gpu_model(ctx, cfg, B, P)

    def run():
        cache = m.kv_cache(B, cfg.seq_len_max)
        out = [m.prefill_kv(cache, prompts)]
        for _ in range(8):
            out.append(m.generate_step_kv(cache)[0])
        cache.destroy()
        return out

    plain = run()
    monkeypatch.setenv("AUR_DEC_PREFETCH", "ofp")
    for blocks in ("32", "7"):
        monkeypatch.setenv("AUR_DEC_PF_BLOCKS", blocks)
        for a, b in zip(plain, run()):
            np.testing.assert_array_equal(a, b)
    m.destroy()


def test_failed_model_create_frees_its_memory(ctx):
    """A model whose activation arena cannot be allocated (max_batch 4096 at
    the config-3 width asks for about a terabyte) fails with the allocator's
    hipErrorOutOfMemory (2), and
    what its constructor had already allocated (parameters, gradients and
    moments, 0.5 GB here) is freed: the device's free memory is back where
    it was, and a model of the same width with a small batch still builds."""
    import ctypes

    from aurora_amd._lib import AuroraError
    from aurora_amd.model import DecoderTransformerGpu

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]

    def free_bytes():
        ctx.sync()
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        assert hip.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
        return f.value

    before = free_bytes()
    for _ in range(3):
        with pytest.raises(AuroraError) as e:
            DecoderTransformerGpu(ctx, 8192, 1024, 2, 16, 4096, 1024, 4096)
        assert e.value.code == 2, e.value  # hipErrorOutOfMemory from hipMalloc
    after = free_bytes()
    assert before - after < (64 << 20), (before, after)
    m = DecoderTransformerGpu(ctx, 8192, 1024, 2, 16, 4096, 1024, 1)
    m.destroy()


def _overfit_model(ctx, seed):
    cfg = OM.Config(vocab=16, d_model=32, n_layer=2, n_head=2, d_ff=64, seq_len_max=16)
    m = _gpu_model(ctx, cfg, 1, OM.init_params(cfg, seed))
    tokens = (np.arange(8) % cfg.vocab).astype(np.uint32)
    return m, tokens, (tokens + 1) % cfg.vocab


def test_muon_hybrid_and_adamw_drop_loss_on_overfit(ctx):
    """tests/gpu_parity.rs:1288-1346 (gpu_muon_hybrid_drops_loss_on_overfit):
    V16 d32 L2 H2 d_ff64, one 8-token sequence whose target is the next id;
    five Muon-hybrid steps (muon lr 0.02, momentum 0.95, Nesterov, NS5;
    AdamW lr 3e-3 without decay on the rest, subset clip 1.0) lower the loss.
    The same with plain AdamW (clip 1.0, lr 3e-3): the loss falls well below
    its start within 30 steps."""
    m, tok, tgt = _overfit_model(ctx, 0x46056)
    m.zero_grad()
    initial = m.train_step(tok, tgt)
    for _ in range(5):
        m.zero_grad()
        m.train_step(tok, tgt)
        m.clip_grads_adamw_subset(1.0)
        m.step_muon_hybrid(muon_lr=0.02, momentum=0.95, nesterov=True, muon_wd=0.0, ns_steps=5,
                           lr=3e-3, weight_decay=0.0)
    m.zero_grad()
    final = m.train_step(tok, tgt)
    m.destroy()
    assert np.isfinite(final) and final < initial, (initial, final)

    m, tok, tgt = _overfit_model(ctx, 0x46057)
    m.zero_grad()
    start = m.train_step(tok, tgt)
    for _ in range(30):
        m.zero_grad()
        m.train_step(tok, tgt)
        m.clip_step_adamw(1.0, lr=3e-3, weight_decay=0.0)
    m.zero_grad()
    end = m.train_step(tok, tgt)
    m.destroy()
    assert np.isfinite(end) and end < 0.5 * start, (start, end)


def test_kv_cache_starts_zeroed_and_reset_matches_fresh(ctx):
    """tests/kv_cache.rs:446-465 (a new cache's K/V history is all zeros,
    current_len 0) and :390-444 (after prefill + steps, reset() zeroes the
    history and current_len, and prefill + step on the reset cache give the
    logits a fresh cache gives — here bit for bit)."""
    cfg = OM.Config(vocab=16, d_model=32, n_layer=2, n_head=2, d_ff=64, seq_len_max=16)
    m = _gpu_model(ctx, cfg, 1, OM.init_params(cfg, 0x9292))
    fresh = m.kv_cache(1, 16)
    assert fresh.current_len == 0
    for layer in range(cfg.n_layer):
        k, v = fresh.history(layer)
        assert not np.any(k) and not np.any(v), layer
    seed_a, seed_b = np.array([[3, 0, 7, 1]], np.uint32), np.array([[5, 2, 9, 11]], np.uint32)
    m.prefill_kv(fresh, seed_b)
    want, _ = m.generate_step_kv(fresh, [8])
    dirty = m.kv_cache(1, 16)
    m.prefill_kv(dirty, seed_a)
    m.generate_step_kv(dirty, [4])
    m.generate_step_kv(dirty, [6])
    dirty.reset()
    assert dirty.current_len == 0
    for layer in range(cfg.n_layer):
        k, v = dirty.history(layer)
        assert not np.any(k) and not np.any(v), layer
    m.prefill_kv(dirty, seed_b)
    got, _ = m.generate_step_kv(dirty, [8])
    np.testing.assert_array_equal(got, want)
    for c in (fresh, dirty):
        c.destroy()
    m.destroy()


def test_gpu_model_matches_torch_definition(ctx):
    """The GPU model against the tiny pre-LN GPT written from torch
    primitives (tests/golden/model_fixture.npz, float64, independent of the
    CPU oracle): logits, per-sequence losses, every gradient of the batch
    mean, one clip + AdamW step with the reference's decay groups, and two
    Muon hybrid steps after the AdamW-subset clip."""
    from pathlib import Path
    fx = np.load(Path(__file__).resolve().parent / "golden" / "model_fixture.npz", allow_pickle=False)
    cfg = OM.Config(*(int(v) for v in fx["cfg"]))

    def tree(prefix):
        P = {k: fx[f"{prefix}.{k}"].astype(np.float32) for k in ("w_tok", "w_pos", "lnf_g", "lnf_b")}
        P["layers"] = [{k: fx[f"{prefix}.l{l}.{k}"].astype(np.float32) for k in OM.LAYER_KEYS}
                       for l in range(cfg.n_layer)]
        return P

    tok, tgt = fx["tokens"], fx["targets"]
    B, T = tok.shape
    P0 = tree("p")
    m = _gpu_model(ctx, cfg, B, P0)
    logits = m.forward(tok).reshape(B, T, cfg.vocab)
    assert fro_rel(logits, fx["logits"]) < 1e-5
    m.zero_grad()
    loss = m.train_step_batch(tok, tgt)
    assert abs(loss - fx["seq_loss"].sum()) < 1e-5 * fx["seq_loss"].sum()
    _compare_tree(m.read_tensors(grad=True), tree("g"), 1e-4, "grad vs torch")
    snap = m.snapshot_state()
    norm = m.clip_grads(float(fx["clip_max_norm"]))
    assert abs(norm - float(fx["grad_norm"])) < 1e-5 * norm
    m.step_adamw(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    got = m.read_tensors(grad=False)
    for (name, l, g), (_, _, w), (_, _, p) in zip(OM.tensors(got), OM.tensors(tree("adamw")), OM.tensors(P0)):
        step, want = g.astype(np.float64) - p.ravel(), w.ravel() - p.ravel().astype(np.float64)
        assert np.max(np.abs(step - want)) < 2e-7 * max(1.0, np.max(np.abs(p))) + 3e-7, (name, l)
    # Muon hybrid from the same gradients and a fresh optimizer state
    m.restore_state(snap)
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    sub = m.clip_grads_adamw_subset(float(fx["subset_max_norm"]))
    assert abs(sub - float(fx["subset_norm"])) < 1e-5 * sub
    prev = P0
    for step in (1, 2):
        m.step_muon_hybrid()
        got = m.read_tensors(grad=False)
        want = tree(f"muon{step}")
        for (name, l, g), (_, _, w), (_, _, p) in zip(OM.tensors(got), OM.tensors(want), OM.tensors(prev)):
            upd = g.astype(np.float64) - p.ravel()
            assert fro_rel(upd, w.ravel() - p.ravel().astype(np.float64)) < 1e-3, (step, name, l)
        prev = got
    m.destroy()
