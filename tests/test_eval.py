"""Forward-only evaluation: per-token NLL (eval_step_batch / eval_step_per_token
/ eval_step, src/gpu/transformer.rs:1723-1811) and the overlapping-window
bits-per-byte caller (examples/aurora_train.rs:1665-1765, src/text_io.rs:43-48).

CPU tests pin the oracle's per-token NLL against closed forms and a float64
log-sum-exp, and the window arithmetic against hand-worked cases and the
every-token-scored-once invariant.  GPU tests compare the device path with
the oracle forward + per-token NLL (tests/gpu_parity.rs:808-818 checks the
same quantity at |Δ| < 5e-2; here 1e-3).
"""
import math

import numpy as np
import pytest
from scipy.special import logsumexp

import oracle as O
from aurora_amd.evaluate import bits_per_byte, cap_windows, eval_windows, evaluate_gpu
from oracle import model as OM

C0 = OM.Config(vocab=256, d_model=128, n_layer=2, n_head=4, d_ff=512, seq_len_max=64)


# ------------------------------------------------------------ oracle pins
def test_token_nll_uniform_logits_is_ln_v():
    for v in (2, 17, 256, 8192):
        t = 5
        logits = np.full((t, v), 3.25, np.float32)
        tgt = np.arange(t, dtype=np.uint32) % v
        nll = O.token_nll(logits, tgt, v)
        np.testing.assert_allclose(nll, math.log(v), rtol=2e-6)


def test_token_nll_clamps_at_1e12():
    v = 8
    logits = np.zeros((2, v), np.float32)
    logits[0, 3] = -200.0  # p_target = e^-200 / (7 + e^-200) < 1e-12
    logits[1, 5] = 200.0   # p_target = 1 exactly in f32
    nll = O.token_nll(logits, np.array([3, 5], np.uint32), v)
    assert nll[0] == np.float32(-math.log(np.float32(1e-12)))
    assert abs(nll[0] - 27.631021) < 1e-5
    assert nll[1] == 0.0


def test_token_nll_matches_float64_logsumexp():
    rng = np.random.default_rng(7)
    t, v = 33, 1000
    logits = (rng.standard_normal((t, v)) * 4).astype(np.float32)
    tgt = rng.integers(0, v, t).astype(np.uint32)
    want = logsumexp(logits.astype(np.float64), axis=1) - logits[np.arange(t), tgt].astype(np.float64)
    got = O.token_nll(logits, tgt, v)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)
    # Its sum is the (pinned) softmax-CE total of the training path.
    total, _ = O.softmax_ce(logits, tgt, v)
    assert abs(float(np.sum(got, dtype=np.float64)) - total) < 1e-4 * total


# ------------------------------------------------------- window arithmetic
def test_eval_windows_hand_cases():
    # stride = 2; starts p with p + 5 < 10.
    assert eval_windows(10, 4) == ([0, 2, 4], 2)
    # Odd seq_len: stride 3, tail 4.
    assert eval_windows(20, 7) == ([0, 3, 6, 9], 4)
    # seq_len 1: stride clamps to 1, tail 0.
    assert eval_windows(5, 1) == ([0, 1, 2], 0)
    # No complete window.
    assert eval_windows(5, 4) == ([], 2)


def test_cap_windows_hand_cases():
    s = list(range(0, 20, 2))  # 10 starts
    assert cap_windows(s, 0) == s
    assert cap_windows(s, 10) == s
    assert cap_windows(s, 3) == [0, 6, 12]   # step 3
    assert cap_windows(s, 4) == [0, 4, 8, 12]  # step 2, first 4
    assert cap_windows(s, 1) == [0]


def test_bits_per_byte_closed_form():
    assert bits_per_byte(0.0, 0) == 0.0
    assert abs(bits_per_byte(math.log(2.0) * 100, 100) - 1.0) < 1e-6
    assert abs(bits_per_byte(12.5, 7) - 12.5 / 7 / math.log(2.0)) < 1e-6


class _PositionModel:
    """Stand-in for the device model: the NLL of a position is its target
    token, and the validation tokens are their own indices, so the summed
    NLL names exactly which validation positions were scored."""

    def __init__(self, max_batch):
        self.max_batch = max_batch
        self.calls = []

    def eval_step_batch(self, inputs, targets):
        inputs, targets = np.asarray(inputs), np.asarray(targets)
        assert inputs.shape == targets.shape and inputs.shape[0] <= self.max_batch
        np.testing.assert_array_equal(targets, inputs + 1)
        self.calls.append(inputs.shape[0])
        return targets.astype(np.float32).ravel()


@pytest.mark.parametrize("n,seq_len,max_batch", [(50, 8, 3), (41, 7, 2), (100, 16, 64), (12, 4, 1)])
def test_evaluate_scores_every_position_once(n, seq_len, max_batch):
    val = np.arange(n, dtype=np.uint32)
    model = _PositionModel(max_batch)
    starts, tail = eval_windows(n, seq_len)
    bpb = evaluate_gpu(model, val, seq_len, comp=1.0)
    last = starts[-1] + seq_len  # last scored target index
    want_nats = sum(range(1, last + 1))
    assert abs(bpb - want_nats / last / math.log(2.0)) < 1e-5 * bpb
    assert sum(model.calls) == len(starts)
    assert all(c == max_batch for c in model.calls[:-1])


def test_evaluate_short_split_is_infinite():
    assert evaluate_gpu(_PositionModel(4), np.arange(9, dtype=np.uint32), 8, 1.0) == math.inf


def test_evaluate_capped_windows_and_compression():
    val = np.arange(200, dtype=np.uint32)
    model = _PositionModel(4)
    starts, tail = cap_windows(eval_windows(200, 10)[0], 5), eval_windows(200, 10)[1]
    want_nats = sum(range(1, 11))
    toks = 10
    for p in starts[1:]:
        want_nats += sum(range(p + 1 + tail, p + 11))
        toks += 10 - tail
    got = evaluate_gpu(model, val, 10, comp=3.7, max_windows=5)
    n_bytes = int(np.float32(toks) * np.float32(3.7))
    assert abs(got - want_nats / n_bytes / math.log(2.0)) < 1e-5 * got


# ------------------------------------------------------------------- GPU
def _gpu_model(ctx, cfg, max_batch, P):
    from aurora_amd.model import DecoderTransformerGpu

    m = DecoderTransformerGpu(ctx, cfg.vocab, cfg.d_model, cfg.n_layer, cfg.n_head, cfg.d_ff,
                              cfg.seq_len_max, max_batch)
    m.load_params(P)
    return m


def _cpu_nll(P, cfg, tok, tgt):
    logits, _ = OM.forward(P, cfg, tok)
    return O.token_nll(logits, tgt, cfg.vocab)


@pytest.mark.gpu
@pytest.mark.parametrize("b,t", [(8, 64), (3, 17), (1, 1)])
def test_eval_step_batch_matches_cpu_per_token(ctx, b, t):
    cfg = C0
    P = OM.init_params(cfg, 0)
    rng = np.random.default_rng(100 + b * t)
    seq = rng.integers(0, cfg.vocab, (b, t + 1)).astype(np.uint32)
    tok, tgt = seq[:, :t].copy(), seq[:, 1:].copy()
    m = _gpu_model(ctx, cfg, 8, P)
    got = m.eval_step_batch(tok, tgt)
    assert got.shape == (b * t,)
    worst = 0.0
    for i in range(b):
        want = _cpu_nll(P, cfg, tok[i], tgt[i])
        err = float(np.max(np.abs(got[i * t:(i + 1) * t] - want)))
        worst = max(worst, err)
        assert err < 1e-3, (i, err)
    print(f"[eval b{b} t{t}] max |nll gpu - cpu| {worst:.2e}")
    # Single-window forms agree with the batched one (M = t instead of b·t
    # may pick another GEMM split, hence a few ulps, not bit identity).
    one = m.eval_step_per_token(tok[b - 1], tgt[b - 1])
    np.testing.assert_allclose(one, got[(b - 1) * t:], rtol=1e-6, atol=1e-5)
    s = m.eval_step(tok[0], tgt[0])
    assert abs(s - float(np.sum(got[:t], dtype=np.float64))) < 1e-5 * max(1.0, abs(s))
    m.destroy()


@pytest.mark.gpu
def test_eval_leaves_params_grads_and_moments_untouched(ctx):
    cfg = C0
    P = OM.init_params(cfg, 1)
    rng = np.random.default_rng(3)
    seq = rng.integers(0, cfg.vocab, (4, 33)).astype(np.uint32)
    tok, tgt = seq[:, :32].copy(), seq[:, 1:].copy()
    m = _gpu_model(ctx, cfg, 4, P)
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    G0 = m.read_tensors(grad=True)
    P0 = m.read_tensors(grad=False)
    nll_a = m.eval_step_batch(tok[::-1].copy(), tgt[::-1].copy())
    for (name, l, g), (_, _, w) in zip(OM.tensors(m.read_tensors(grad=True)), OM.tensors(G0)):
        np.testing.assert_array_equal(g, w, err_msg=f"grad {name} {l}")
    for (name, l, g), (_, _, w) in zip(OM.tensors(m.read_tensors(grad=False)), OM.tensors(P0)):
        np.testing.assert_array_equal(g, w, err_msg=f"param {name} {l}")
    # Eval between the backward and the optimizer step changes nothing about
    # the step: the update equals the one without the eval call.
    m.clip_grads(1.0)
    m.step_adamw(lr=3e-4, weight_decay=0.1)
    P1 = m.read_tensors(grad=False)
    m2 = _gpu_model(ctx, cfg, 4, P)
    m2.zero_grad()
    m2.train_step_batch(tok, tgt)
    m2.clip_grads(1.0)
    m2.step_adamw(lr=3e-4, weight_decay=0.1)
    for (name, l, g), (_, _, w) in zip(OM.tensors(P1), OM.tensors(m2.read_tensors(grad=False))):
        np.testing.assert_array_equal(g, w, err_msg=f"stepped param {name} {l}")
    # Repeat evals of the same parameters are bit-identical.
    m3 = _gpu_model(ctx, cfg, 4, P)
    np.testing.assert_array_equal(nll_a, m3.eval_step_batch(tok[::-1].copy(), tgt[::-1].copy()))
    np.testing.assert_array_equal(m.eval_step_batch(tok, tgt), m.eval_step_batch(tok, tgt))
    m3.destroy()
    m.destroy()
    m2.destroy()


@pytest.mark.gpu
def test_eval_rejects_bad_input(ctx):
    from aurora_amd._lib import AuroraError

    cfg = C0
    m = _gpu_model(ctx, cfg, 2, OM.init_params(cfg, 0))
    tok = np.zeros((3, 8), np.uint32)
    with pytest.raises(AuroraError):
        m.eval_step_batch(tok, tok)  # b > max_batch
    with pytest.raises(AuroraError):
        m.eval_step_batch(np.zeros((1, 65), np.uint32), np.zeros((1, 65), np.uint32))  # t > seq_len_max
    bad = np.zeros((1, 8), np.uint32)
    bad[0, 3] = cfg.vocab
    with pytest.raises(AuroraError):
        m.eval_step_batch(np.zeros((1, 8), np.uint32), bad)  # target out of vocab
    assert m.eval_step_batch([], []).size == 0
    m.destroy()


@pytest.mark.gpu
def test_evaluate_gpu_bpb_matches_cpu_evaluate(ctx):
    """Sliding-window BPB on the device vs the CPU evaluate's per-window
    logsumexp scoring (examples/aurora_train.rs:1691-1725) over the oracle."""
    cfg = C0
    P = OM.init_params(cfg, 2)
    rng = np.random.default_rng(11)
    val = rng.integers(0, cfg.vocab, 700).astype(np.uint32)
    seq_len, comp = 64, 2.5
    m = _gpu_model(ctx, cfg, 8, P)
    got = evaluate_gpu(m, val, seq_len, comp)
    starts, tail = eval_windows(val.size, seq_len)
    nats, toks = 0.0, 0
    for wi, p in enumerate(starts):
        sf = 0 if wi == 0 else tail
        nll = _cpu_nll(P, cfg, val[p:p + seq_len], val[p + 1:p + seq_len + 1])
        nats += float(np.sum(nll[sf:], dtype=np.float64))
        toks += seq_len - sf
    want = nats / int(toks * comp) / math.log(2.0)
    print(f"[evaluate] bpb gpu {got:.6f} cpu {want:.6f} over {len(starts)} windows")
    assert abs(got - want) < 1e-4 * want
    m.destroy()
