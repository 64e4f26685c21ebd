"""GPU parity of causal MHA forward / backward and KV-cache decode attention.

Mirrors tests/gpu_parity.rs:217-355 (causal_mha_{forward,backward}_matches_cpu,
shapes (t,H,dh) ∈ {(4,2,8),(8,4,16),(12,2,32)} and t=6,H=2,dh=8) against the
CPU restatement, tests/kv_cache.rs:346-386 (t_total = 80 > 64: stride loops),
then the BASELINE config-2 shape (B16 H8 T1024 dh64) against float64.
North-star tolerance for attention: 1e-3 (normalised, see parity.py).
"""
import numpy as np
import pytest

import oracle
from tests.attn_ref import causal_attention_f64, causal_attention_grad_f64
from tests.parity import fro_rel, max_norm_rel, max_rel_err

pytestmark = pytest.mark.gpu

TOL_ATTN = 1e-3
TOL_REF = 5e-2  # tests/gpu_parity.rs:255, :350 (pointwise vs the fp32 CPU path)


def _n(rng, n):
    return rng.standard_normal(n).astype(np.float32)


def _fwd(ctx, q, k, v, B, T, H, dh):
    from aurora_amd.gpu import CausalMhaForwardKernel, GpuBuffer

    bq, bk, bv = (GpuBuffer.from_slice(ctx, x) for x in (q, k, v))
    out = GpuBuffer.zeros(ctx, B * T * H * dh)
    lse = GpuBuffer.zeros(ctx, B * H * T)
    CausalMhaForwardKernel.new(ctx).dispatch_into(ctx, bq, bk, bv, out, lse, T, H, dh, b=B)
    res = out.download(), lse.download()
    for x in (bq, bk, bv, out, lse):
        x.free()
    return res


def _bwd(ctx, q, k, v, o, lse, d_out, B, T, H, dh, init=None):
    from aurora_amd.gpu import CausalMhaBackwardKernel, GpuBuffer

    n = B * T * H * dh
    bufs = [GpuBuffer.from_slice(ctx, x) for x in (q, k, v, o, lse, d_out)]
    if init is None:
        grads = [GpuBuffer.zeros(ctx, n) for _ in range(3)]
    else:
        grads = [GpuBuffer.from_slice(ctx, x) for x in init]
    ws = GpuBuffer.empty(ctx, CausalMhaBackwardKernel.workspace_len(T, H, B))
    CausalMhaBackwardKernel.new(ctx).dispatch_into(ctx, *bufs, *grads, ws, T, H, dh, b=B)
    res = [g.download() for g in grads]
    for x in bufs + grads + [ws]:
        x.free()
    return res


@pytest.mark.parametrize("t,H,dh", [(4, 2, 8), (8, 4, 16), (12, 2, 32), (70, 2, 64), (129, 3, 32),
                                    (33, 2, 24), (70, 3, 40), (65, 2, 48), (100, 2, 56)])
def test_causal_mha_forward_matches_cpu(ctx, t, H, dh):
    rng = np.random.default_rng(0x4274 + t)
    d = H * dh
    q, k, v = _n(rng, t * d), _n(rng, t * d), _n(rng, t * d)
    out, lse = _fwd(ctx, q, k, v, 1, t, H, dh)
    want, _ = oracle.mha_heads_forward(q, k, v, t, H, dh)
    assert max_rel_err(out, want) < TOL_REF
    o64, l64 = causal_attention_f64(*(x.reshape(1, t, H, dh).astype(np.float64) for x in (q, k, v)))
    assert fro_rel(out, o64) < TOL_ATTN and max_norm_rel(out, o64) < TOL_ATTN
    np.testing.assert_allclose(lse.reshape(1, H, t), l64, rtol=0, atol=1e-4)


@pytest.mark.parametrize("t,H,dh", [(6, 2, 8), (12, 2, 32), (65, 2, 64), (200, 1, 16),
                                    (33, 2, 24), (90, 1, 40), (70, 2, 48), (65, 2, 56)])
def test_causal_mha_backward_matches_cpu(ctx, t, H, dh):
    """gpu_parity.rs:267-355: dq/dk/dv accumulate into zeroed buffers.  The
    reference's kernels take any d_head ≤ 64 (src/gpu/attention.rs:249-331);
    here every multiple of 8 is covered, 24/40/48/56 with their last 16-wide
    head chunk half empty."""
    rng = np.random.default_rng(0x5151 + t)
    d = H * dh
    q, k, v, do = (_n(rng, t * d) for _ in range(4))
    out, lse = _fwd(ctx, q, k, v, 1, t, H, dh)
    dq, dk, dv = _bwd(ctx, q, k, v, out, lse, do, 1, t, H, dh)
    _, probs = oracle.mha_heads_forward(q, k, v, t, H, dh)
    wq, wk, wv = oracle.mha_heads_backward(q, k, v, probs, do, t, H, dh)
    for got, want in ((dq, wq), (dk, wk), (dv, wv)):
        assert fro_rel(got, want) < TOL_ATTN
    g64 = causal_attention_grad_f64(*(x.reshape(1, t, H, dh).astype(np.float64) for x in (q, k, v, do)))
    for got, want in zip((dq, dk, dv), g64):
        assert fro_rel(got, want) < TOL_ATTN and max_norm_rel(got, want) < TOL_ATTN


_RAND_ATTN = [(int(r.integers(1, 4)), int(r.integers(1, 330)), int(r.integers(1, 5)), int(r.choice([8, 16, 32, 64])))
              for r in (np.random.default_rng(7700 + i) for i in range(8))]


@pytest.mark.parametrize("B,t,H,dh", _RAND_ATTN)
def test_seeded_random_batched_forward_backward(ctx, B, t, H, dh):
    """8 seeded random (batch, t, heads, d_head): ragged last tiles, every
    d_head, batch > 1; forward, LSE and all three gradients against float64."""
    rng = np.random.default_rng(B * 100_003 + t * 101 + H * 7 + dh)
    n = B * t * H * dh
    q, k, v, do = (_n(rng, n) for _ in range(4))
    out, lse = _fwd(ctx, q, k, v, B, t, H, dh)
    shp = (B, t, H, dh)
    o64, l64 = causal_attention_f64(*(x.reshape(shp).astype(np.float64) for x in (q, k, v)))
    assert fro_rel(out, o64) < TOL_ATTN and max_norm_rel(out, o64) < TOL_ATTN
    np.testing.assert_allclose(lse.reshape(B, H, t), l64, rtol=0, atol=1e-4)
    grads = _bwd(ctx, q, k, v, out, lse, do, B, t, H, dh)
    g64 = causal_attention_grad_f64(*(x.reshape(shp).astype(np.float64) for x in (q, k, v, do)))
    for got, want in zip(grads, g64):
        assert fro_rel(got, want) < TOL_ATTN and max_norm_rel(got, want) < TOL_ATTN


@pytest.mark.parametrize("env", ["AUR_ATTN_FWD_STAGED", "AUR_ATTN_DKV_NS2", "AUR_ATTN_DQ_STAGED"])
def test_alternate_kernels_d64(ctx, monkeypatch, env):
    """The d_head = 64 kernels reachable only through the overrides (register-
    staged forward, two-stage dK/dV ring, register-staged dQ) against float64,
    ragged T, batch 2."""
    monkeypatch.setenv(env, "1")
    B, t, H, dh = 2, 201, 3, 64
    rng = np.random.default_rng(4242 + len(env))
    n = B * t * H * dh
    q, k, v, do = (_n(rng, n) for _ in range(4))
    out, lse = _fwd(ctx, q, k, v, B, t, H, dh)
    shp = (B, t, H, dh)
    o64, l64 = causal_attention_f64(*(x.reshape(shp).astype(np.float64) for x in (q, k, v)))
    assert fro_rel(out, o64) < TOL_ATTN and max_norm_rel(out, o64) < TOL_ATTN
    grads = _bwd(ctx, q, k, v, out, lse, do, B, t, H, dh)
    g64 = causal_attention_grad_f64(*(x.reshape(shp).astype(np.float64) for x in (q, k, v, do)))
    for got, want in zip(grads, g64):
        assert fro_rel(got, want) < TOL_ATTN and max_norm_rel(got, want) < TOL_ATTN


def test_backward_accumulates_and_is_deterministic(ctx):
    B, T, H, dh = 2, 97, 2, 64
    rng = np.random.default_rng(9)
    n = B * T * H * dh
    q, k, v, do = (_n(rng, n) for _ in range(4))
    init = [_n(rng, n) for _ in range(3)]
    out, lse = _fwd(ctx, q, k, v, B, T, H, dh)
    g0 = _bwd(ctx, q, k, v, out, lse, do, B, T, H, dh)
    g1 = _bwd(ctx, q, k, v, out, lse, do, B, T, H, dh, init=init)
    g2 = _bwd(ctx, q, k, v, out, lse, do, B, T, H, dh, init=init)
    for a0, a1, a2, i0 in zip(g0, g1, g2, init):
        assert np.array_equal(a1, a2)  # bitwise run-to-run
        np.testing.assert_allclose(a1, i0 + a0, rtol=1e-5, atol=1e-5)


def test_causal_future_independence(ctx):
    """tests/transformer_primitives.rs:179: changing k/v at j > i leaves out[i]."""
    B, T, H, dh = 1, 150, 2, 64
    rng = np.random.default_rng(11)
    n = T * H * dh
    q, k, v = _n(rng, n), _n(rng, n), _n(rng, n)
    o1, _ = _fwd(ctx, q, k, v, B, T, H, dh)
    cut = 77
    k2, v2 = k.copy(), v.copy()
    k2[(cut + 1) * H * dh:] = _n(rng, n - (cut + 1) * H * dh)
    v2[(cut + 1) * H * dh:] = _n(rng, n - (cut + 1) * H * dh)
    o2, _ = _fwd(ctx, q, k2, v2, B, T, H, dh)
    m = (cut + 1) * H * dh
    assert np.array_equal(o1[:m], o2[:m])
    assert not np.array_equal(o1[m:], o2[m:])


def test_config2_mha_fwd_bwd(ctx):
    """B16 H8 T1024 dh64, N(0,1) seed 1, scale 1/8, causal."""
    B, T, H, dh = 16, 1024, 8, 64
    rng = np.random.default_rng(1)
    n = B * T * H * dh
    q, k, v, do = (_n(rng, n) for _ in range(4))
    out, lse = _fwd(ctx, q, k, v, B, T, H, dh)
    dq, dk, dv = _bwd(ctx, q, k, v, out, lse, do, B, T, H, dh)
    shp = (B, T, H, dh)
    q64, k64, v64, do64 = (x.reshape(shp).astype(np.float64) for x in (q, k, v, do))
    o64, l64 = causal_attention_f64(q64, k64, v64)
    assert fro_rel(out, o64) < TOL_ATTN and max_norm_rel(out, o64) < TOL_ATTN
    assert np.max(np.abs(lse.reshape(B, H, T) - l64)) < 1e-4
    for got, want in zip((dq, dk, dv), causal_attention_grad_f64(q64, k64, v64, do64)):
        assert fro_rel(got, want) < TOL_ATTN and max_norm_rel(got, want) < TOL_ATTN


# ------------------------------------------------------------------ KV decode
def _kv_single(ctx, q_new, kh, vh, t_total, H, dh, max_len):
    from aurora_amd.gpu import GpuBuffer, MhaKvCacheKernel

    bq, bk, bv = (GpuBuffer.from_slice(ctx, x) for x in (q_new, kh, vh))
    out = GpuBuffer.zeros(ctx, H * dh)
    scratch = GpuBuffer.empty(ctx, MhaKvCacheKernel.scratch_len(H, max_len))
    MhaKvCacheKernel.new(ctx).dispatch_into(ctx, bq, bk, bv, out, scratch, t_total, H, dh, max_len)
    res = out.download()
    for x in (bq, bk, bv, out, scratch):
        x.free()
    return res


@pytest.mark.parametrize("t_total,H,dh", [(1, 2, 16), (5, 2, 16), (64, 2, 32), (80, 2, 16),
                                          (129, 4, 64), (300, 1, 8), (513, 16, 64),
                                          (100, 2, 24), (70, 2, 40), (129, 3, 48), (65, 2, 56)])
def test_mha_kv_step_matches_cpu(ctx, t_total, H, dh):
    """tests/kv_cache.rs:346-386 covers t_total=80 > 64 (stride loops)."""
    rng = np.random.default_rng(100 + t_total)
    d, max_len = H * dh, max(t_total, 96)
    q_new = _n(rng, d)
    kh, vh = _n(rng, max_len * d), _n(rng, max_len * d)
    got = _kv_single(ctx, q_new, kh, vh, t_total, H, dh, max_len)
    want = oracle.kv_attend(q_new, kh, vh, t_total, H, dh)
    assert fro_rel(got, want) < TOL_ATTN and max_norm_rel(got, want) < TOL_ATTN


def test_kv_step_equals_last_row_of_full_forward(ctx):
    """The decode step's query against the cache equals the full causal
    forward's last row (tests/kv_cache.rs:64-138 property, kernel level)."""
    T, H, dh = 200, 4, 64
    rng = np.random.default_rng(21)
    d = H * dh
    q, k, v = _n(rng, T * d), _n(rng, T * d), _n(rng, T * d)
    out, _ = _fwd(ctx, q, k, v, 1, T, H, dh)
    for t in (1, 64, 65, 128, 200):
        got = _kv_single(ctx, q[(t - 1) * d:t * d], k, v, t, H, dh, T)
        np.testing.assert_allclose(got, out.reshape(T, d)[t - 1], rtol=0, atol=2e-5)


def test_kv_step_batched_ragged_lengths(ctx):
    from aurora_amd.gpu import GpuBuffer, MhaKvCacheKernel

    B, H, dh, max_len = 5, 4, 64, 300
    rng = np.random.default_rng(31)
    d = H * dh
    lens = np.array([1, 64, 129, 300, 257], np.int32)
    q_new = _n(rng, B * d)
    kh, vh = _n(rng, B * max_len * d), _n(rng, B * max_len * d)
    bq, bk, bv = (GpuBuffer.from_slice(ctx, x) for x in (q_new, kh, vh))
    bt = GpuBuffer.from_slice(ctx, lens)
    out = GpuBuffer.zeros(ctx, B * d)
    scratch = GpuBuffer.empty(ctx, MhaKvCacheKernel.scratch_len(H, max_len, B))
    MhaKvCacheKernel.new(ctx).dispatch_batched(ctx, bq, bk, bv, out, scratch, bt, int(lens.max()),
                                               B, H, dh, max_len)
    got = out.download().reshape(B, d)
    for i in range(B):
        want = oracle.kv_attend(q_new[i * d:(i + 1) * d], kh[i * max_len * d:(i + 1) * max_len * d],
                                vh[i * max_len * d:(i + 1) * max_len * d], int(lens[i]), H, dh)
        assert fro_rel(got[i], want) < TOL_ATTN, i


@pytest.mark.parametrize("dh", [8, 16, 24, 32, 40, 48, 56, 64])
def test_kv_step_batched_one_block_per_head(ctx, dh, monkeypatch):
    """B·H ≥ CU count takes the single-launch path (a block per sequence and
    head, waves merged in LDS).  Ragged lengths including 1 and max_len,
    against the oracle per sequence, against the chunked two-launch path,
    and bit-identical on a repeat."""
    from aurora_amd.gpu import GpuBuffer, MhaKvCacheKernel

    B, max_len = 32, 700
    H = 256 // B * (2 if dh <= 16 else 1)
    d = H * dh
    rng = np.random.default_rng(41 + dh)
    lens = rng.integers(1, max_len + 1, B).astype(np.int32)
    lens[0], lens[1], lens[2] = 1, max_len, 2
    t_max = int(lens.max())
    q_new = _n(rng, B * d)
    kh, vh = _n(rng, B * max_len * d), _n(rng, B * max_len * d)
    bq, bk, bv = (GpuBuffer.from_slice(ctx, x) for x in (q_new, kh, vh))
    bt = GpuBuffer.from_slice(ctx, lens)
    scratch = GpuBuffer.empty(ctx, MhaKvCacheKernel.scratch_len(H, max_len, B))
    kern = MhaKvCacheKernel.new(ctx)

    def run():
        out = GpuBuffer.zeros(ctx, B * d)
        kern.dispatch_batched(ctx, bq, bk, bv, out, scratch, bt, t_max, B, H, dh, max_len)
        return out.download().reshape(B, d)

    got = run()
    np.testing.assert_array_equal(run(), got)
    for i in range(B):
        want = oracle.kv_attend(q_new[i * d:(i + 1) * d], kh[i * max_len * d:(i + 1) * max_len * d],
                                vh[i * max_len * d:(i + 1) * max_len * d], int(lens[i]), H, dh)
        assert fro_rel(got[i], want) < TOL_ATTN, i
        assert max_rel_err(got[i], want) < TOL_REF, i
    monkeypatch.setenv("AUR_KV_CHUNKED", "1")
    chunked = run()
    assert fro_rel(got, chunked) < 1e-5


def test_config2_probability_rows_sum_to_one_and_lse(ctx):
    """Size-free invariants at the config-2 shape (B16 H8 T1024 dh64): with
    V = 1 every output is Σ_j P_ij = 1 exactly up to rounding (rows of P sum
    to one), and with K = 0 every score is 0, so row i attends uniformly over
    its i + 1 keys: lse_i = ln(i + 1) and O = the running mean of V."""
    B, T, H, dh = 16, 1024, 8, 64
    n = B * T * H * dh
    rng = np.random.default_rng(3)
    q, k = _n(rng, n), _n(rng, n)
    ones = np.ones(n, np.float32)
    o, _ = _fwd(ctx, q, k, ones, B, T, H, dh)
    assert np.max(np.abs(o - 1.0)) < 1e-5, np.max(np.abs(o - 1.0))
    v = _n(rng, n)
    o, lse = _fwd(ctx, q, np.zeros(n, np.float32), v, B, T, H, dh)
    want_lse = np.log(np.arange(1, T + 1, dtype=np.float64))
    assert np.max(np.abs(lse.reshape(B, H, T) - want_lse)) < 1e-4
    v4 = v.reshape(B, T, H, dh).astype(np.float64)
    running = np.cumsum(v4, axis=1) / np.arange(1, T + 1)[None, :, None, None]
    assert fro_rel(o.reshape(B, T, H, dh), running) < 1e-5


def test_config2_zero_output_gradient_gives_zero_gradients(ctx):
    """dO = 0 ⇒ dQ = dK = dV = 0 (every backward term carries dO or dP = dO·Vᵀ),
    and the accumulate contract leaves non-zero destinations unchanged."""
    B, T, H, dh = 4, 1024, 8, 64
    n = B * T * H * dh
    rng = np.random.default_rng(4)
    q, k, v = _n(rng, n), _n(rng, n), _n(rng, n)
    o, lse = _fwd(ctx, q, k, v, B, T, H, dh)
    init = [_n(rng, n) for _ in range(3)]
    dq, dk, dv = _bwd(ctx, q, k, v, o, lse, np.zeros(n, np.float32), B, T, H, dh, init=init)
    for got, want in zip((dq, dk, dv), init):
        np.testing.assert_array_equal(got, want)


# ------------------------------- the reference's own scratch allocations
CANARY = 4096  # floats of guard on each side (16 KB: keeps the region 16-byte aligned)


def _guarded(ctx, n):
    """A device region of exactly n floats inside a larger allocation whose
    two guard regions hold a known pattern: (buffer, view of the region)."""
    from aurora_amd.gpu import GpuBuffer

    host = np.full(CANARY + n + CANARY, 1234.5, np.float32)
    host[CANARY:CANARY + n] = 0.0
    buf = GpuBuffer.from_slice(ctx, host)
    return buf, GpuBuffer(ctx, buf.ptr + 4 * CANARY, n)


def _guards_intact(buf, n):
    host = buf.download()
    return bool(np.all(host[:CANARY] == 1234.5) and np.all(host[CANARY + n:] == 1234.5))


@pytest.mark.parametrize("t,H,dh", [(6, 2, 8), (64, 2, 64), (65, 2, 16), (1, 1, 8)])
def test_backward_within_reference_d_scores_allocation(ctx, t, H, dh):
    """The reference allocates the backward's d_scores scratch as exactly
    n_head·t·t floats (tests/gpu_parity.rs:292-297, src/gpu/transformer.rs:
    314, 375): at its own parity case (t = 6, H = 2, d_head = 8: 72 floats)
    and at short or ragged t, where the tiled dS layout needs more than that,
    the call writes nothing outside those floats and matches the oracle."""
    from aurora_amd.gpu import CausalMhaBackwardKernel, GpuBuffer

    d = H * dh
    rng = np.random.default_rng(0xB17D + t)
    q, k, v, dy = (_n(rng, t * d) for _ in range(4))
    o, lse = _fwd(ctx, q, k, v, 1, t, H, dh)
    n_ws = H * t * t
    assert CausalMhaBackwardKernel.workspace_len(t, H) <= n_ws
    guard, ws = _guarded(ctx, n_ws)
    bufs = [GpuBuffer.from_slice(ctx, x) for x in (q, k, v, o, lse, dy)]
    grads = [GpuBuffer.zeros(ctx, t * d) for _ in range(3)]
    CausalMhaBackwardKernel.new(ctx).dispatch_into(ctx, *bufs, *grads, ws, t, H, dh)
    got = [g.download() for g in grads]
    assert _guards_intact(guard, n_ws)
    _, probs = oracle.mha_heads_forward(q, k, v, t, H, dh)
    want = oracle.mha_heads_backward(q, k, v, probs, dy, t, H, dh)
    g64 = causal_attention_grad_f64(*(x.reshape(1, t, H, dh).astype(np.float64) for x in (q, k, v, dy)))
    for g, w, w64 in zip(got, want, g64):
        # (row 0's dq is 0 in exact arithmetic: normalised metrics, as above)
        assert fro_rel(g, w) < TOL_ATTN and max_norm_rel(g, w) < TOL_ATTN
        assert fro_rel(g, w64) < TOL_ATTN and max_norm_rel(g, w64) < TOL_ATTN


@pytest.mark.parametrize("max_len,t_total,H,dh", [(64, 64, 2, 64), (64, 17, 4, 32), (130, 130, 2, 64),
                                                  (130, 100, 2, 16), (256, 200, 3, 64)])
def test_kv_step_within_reference_scratch_allocation(ctx, max_len, t_total, H, dh):
    """MhaKvCacheKernel's scratch is n_head·max_len floats in the reference
    (src/gpu/transformer.rs:2432); the tiny preset decodes with max_len 64
    (src/transformer/model.rs:108).  With exactly that allocation nothing is
    written outside it, and the result matches the oracle (max_len 64 and 130
    take the scratch-free kernel; 256 has room for the chunk records)."""
    from aurora_amd.gpu import GpuBuffer, MhaKvCacheKernel

    d = H * dh
    rng = np.random.default_rng(max_len + t_total)
    q_new = _n(rng, d)
    kh, vh = _n(rng, max_len * d), _n(rng, max_len * d)
    n_s = H * max_len
    assert MhaKvCacheKernel.scratch_len(H, max_len) <= n_s
    guard, scratch = _guarded(ctx, n_s)
    bq, bk, bv = (GpuBuffer.from_slice(ctx, x) for x in (q_new, kh, vh))
    out = GpuBuffer.zeros(ctx, d)
    MhaKvCacheKernel.new(ctx).dispatch_into(ctx, bq, bk, bv, out, scratch, t_total, H, dh, max_len)
    got = out.download()
    assert _guards_intact(guard, n_s)
    want = oracle.kv_attend(q_new, kh, vh, t_total, H, dh)
    assert fro_rel(got, want) < TOL_ATTN and max_norm_rel(got, want) < TOL_ATTN


# ------------------------------------------------ any d_head (the reference's)
@pytest.mark.parametrize("B,t,H,dh", [(1, 6, 2, 1), (2, 37, 3, 12), (1, 70, 2, 20), (2, 65, 1, 36), (1, 9, 4, 60),
                                      (1, 130, 2, 63)])
def test_forward_backward_any_d_head(ctx, B, t, H, dh):
    """The reference's training kernels take any d_head ≤ 64 (one thread per
    column with a guard, src/gpu/attention.rs:266-331); here d_head that is
    not a multiple of 8 runs through zero-padded heads.  Forward, LSE and
    the accumulated gradients (onto non-zero destinations) against float64."""
    rng = np.random.default_rng(B * 1000 + t * 10 + dh)
    n = B * t * H * dh
    q, k, v, do = (_n(rng, n) for _ in range(4))
    out, lse = _fwd(ctx, q, k, v, B, t, H, dh)
    shp = (B, t, H, dh)
    o64, l64 = causal_attention_f64(*(x.reshape(shp).astype(np.float64) for x in (q, k, v)))
    assert fro_rel(out, o64) < TOL_ATTN and max_norm_rel(out, o64) < TOL_ATTN
    np.testing.assert_allclose(lse.reshape(B, H, t), l64, rtol=0, atol=1e-4)
    init = [_n(rng, n) for _ in range(3)]
    grads = _bwd(ctx, q, k, v, out, lse, do, B, t, H, dh, init=init)
    g64 = causal_attention_grad_f64(*(x.reshape(shp).astype(np.float64) for x in (q, k, v, do)))
    for got, want, base in zip(grads, g64, init):
        d = got.astype(np.float64) - base
        assert fro_rel(d, want) < TOL_ATTN and max_norm_rel(d, want) < TOL_ATTN


def test_kv_step_generic_beyond_16384_keys_refused(ctx):
    """The generic KV kernel keeps a sequence's scores in LDS: a history past
    16384 keys with a d_head it serves is refused (AUR_ELIMIT) before launch."""
    from aurora_amd._lib import AuroraError

    H, dh, t = 1, 12, 16385
    z = np.zeros(t * H * dh, np.float32)
    with pytest.raises(AuroraError) as e:
        _kv_single(ctx, np.zeros(H * dh, np.float32), z, z, t, H, dh, t)
    assert e.value.code == 10003


def test_any_d_head_beyond_64_refused(ctx):
    from aurora_amd._lib import AuroraError

    with pytest.raises(AuroraError) as e:
        _fwd(ctx, *(np.zeros(4 * 2 * 72, np.float32) for _ in range(3)), 1, 4, 2, 72)
    assert e.value.code == 10003


@pytest.mark.parametrize("t_total,H,dh,max_len", [(5, 2, 12, 8), (80, 3, 20, 96), (129, 2, 100, 130),
                                                  (300, 1, 128, 300), (64, 4, 6, 64), (33, 2, 1, 40),
                                                  (16384, 1, 12, 16384)])
def test_kv_step_any_d_head(ctx, t_total, H, dh, max_len):
    """src/gpu/kv_cache.rs:339-348 stride-loops over d_head, past 64 too:
    d_head that the bandwidth-shaped kernels do not take runs the generic
    kernel (up to 16384 keys, its LDS score buffer, which the last case
    fills); against the oracle."""
    d = H * dh
    rng = np.random.default_rng(t_total * 7 + dh)
    q_new = _n(rng, d)
    kh, vh = _n(rng, max_len * d), _n(rng, max_len * d)
    got = _kv_single(ctx, q_new, kh, vh, t_total, H, dh, max_len)
    want = oracle.kv_attend(q_new, kh, vh, t_total, H, dh)
    assert fro_rel(got, want) < TOL_ATTN and max_norm_rel(got, want) < TOL_ATTN
