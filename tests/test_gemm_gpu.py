"""GPU parity of the GEMM family (A@B, A@Bᵀ, dest += dYᵀ·X) through the C ABI.

Mirrors tests/gpu_parity.rs:57-109 (gemm / gemm_transpose_b) and :469-508
(outer_product_accum with a non-zero initial dest) at the reference's own
tiny shapes against the CPU restatement, then the BASELINE config-1 sweep
(M = 8192) against a float64 product with normalised gates (see parity.py).
"""
import numpy as np
import pytest

import oracle
from tests.parity import componentwise, fro_rel, max_rel_err

pytestmark = pytest.mark.gpu

TOL_GEMM = 1e-4  # <= 1e-4 per GEMM (normalised, vs float64)
TOL_REF = 5e-3   # tests/gpu_parity.rs:81, pointwise vs the fp32 CPU oracle


def _u(rng, n):
    return rng.uniform(-1.0, 1.0, n).astype(np.float32)


def _run(ctx, fn, a, b, c_len, *dims, c_init=None):
    from aurora_amd.gpu import GpuBuffer

    ab = GpuBuffer.from_slice(ctx, a)
    bb = GpuBuffer.from_slice(ctx, b)
    cb = GpuBuffer.from_slice(ctx, c_init) if c_init is not None else GpuBuffer.zeros(ctx, c_len)
    fn(ctx, ab, bb, cb, *dims)
    out = cb.download()
    for x in (ab, bb, cb):
        x.free()
    return out


def _nn(ctx, a, b, m, n, k):
    from aurora_amd.gpu import GemmKernel

    return _run(ctx, GemmKernel.new(ctx).dispatch_into, a, b, m * n, m, n, k)


def _nt(ctx, a, b, m, n, k):
    from aurora_amd.gpu import GemmTransposeBKernel

    return _run(ctx, GemmTransposeBKernel.new(ctx).dispatch_into, a, b, m * n, m, n, k)


def _outer(ctx, x, dy, dest, d_out, d_in, t):
    from aurora_amd.gpu import OuterProductAccumKernel

    return _run(ctx, OuterProductAccumKernel.new(ctx).dispatch_into, x, dy, d_out * d_in,
                d_out, d_in, t, c_init=dest)


def _gates(c, a64, b64, c0=None):
    """Componentwise + Frobenius error of c against the float64 product."""
    c64 = a64 @ b64
    bound = np.abs(a64) @ np.abs(b64)
    if c0 is not None:
        c64 = c64 + c0
        bound = bound + np.abs(c0)
    c = c.reshape(c64.shape)
    return componentwise(c, c64, bound), fro_rel(c, c64)


@pytest.mark.parametrize("m,k,n", [(16, 16, 16), (33, 64, 17), (8, 128, 64), (64, 32, 96)])
def test_gemm_matches_cpu(ctx, m, k, n):
    """tests/gpu_parity.rs:57-82 shapes."""
    rng = np.random.default_rng(1000 + m + k + n)
    a, b = _u(rng, m * k), _u(rng, k * n)
    got = _nn(ctx, a, b, m, n, k)
    want = oracle.cpu_gemm(a, b, m, k, n)
    assert max_rel_err(got, want) < TOL_REF
    cw, fr = _gates(got, a.reshape(m, k).astype(np.float64), b.reshape(k, n).astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)


@pytest.mark.parametrize("m,k,n", [(16, 16, 16), (32, 48, 20), (8, 64, 64)])
def test_gemm_transpose_b_matches_cpu(ctx, m, k, n):
    """tests/gpu_parity.rs:84-109 shapes."""
    rng = np.random.default_rng(2000 + m + k + n)
    a, b = _u(rng, m * k), _u(rng, n * k)
    got = _nt(ctx, a, b, m, n, k)
    want = oracle.cpu_gemm_transpose_b(a, b, m, k, n)
    assert max_rel_err(got, want) < TOL_REF
    cw, fr = _gates(got, a.reshape(m, k).astype(np.float64), b.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)


@pytest.mark.parametrize("d_out,d_in,t", [(16, 16, 8), (32, 64, 12), (8, 24, 16)])
def test_outer_product_accum_matches_cpu(ctx, d_out, d_in, t):
    """tests/gpu_parity.rs:469-508: accumulate into a NON-ZERO dest."""
    rng = np.random.default_rng(3000 + d_out + d_in + t)
    x, dy, dest = _u(rng, t * d_in), _u(rng, t * d_out), _u(rng, d_out * d_in)
    got = _outer(ctx, x, dy, dest, d_out, d_in, t)
    want = dest.copy()
    oracle.outer_accum(x, dy, want, d_out, d_in, t)
    assert max_rel_err(got, want) < TOL_REF
    cw, fr = _gates(got, dy.reshape(t, d_out).T.astype(np.float64),
                    x.reshape(t, d_in).astype(np.float64), dest.reshape(d_out, d_in))
    assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (130, 33, 70), (257, 1000, 129), (3, 7, 5),
                                   (128, 2048, 128), (64, 4096, 8)])
def test_ragged_shapes_all_forms(ctx, m, k, n):
    """Edge tiles, K tails, non-multiple-of-4 strides (scalar load path),
    and split-K at long K with a small output."""
    rng = np.random.default_rng(4000 + m * 7 + k * 3 + n)
    a = _u(rng, m * k)
    b_nn = _u(rng, k * n)
    b_nt = _u(rng, n * k)
    a64 = a.reshape(m, k).astype(np.float64)
    cw, fr = _gates(_nn(ctx, a, b_nn, m, n, k), a64, b_nn.reshape(k, n).astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nn", cw, fr)
    cw, fr = _gates(_nt(ctx, a, b_nt, m, n, k), a64, b_nt.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nt", cw, fr)
    # outer accum with d_out = m, d_in = n, t = k
    x, dy, dest = _u(rng, k * n), _u(rng, k * m), _u(rng, m * n)
    got = _outer(ctx, x, dy, dest, m, n, k)
    cw, fr = _gates(got, dy.reshape(k, m).T.astype(np.float64), x.reshape(k, n).astype(np.float64),
                    dest.reshape(m, n))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("outer", cw, fr)


_RAND_SHAPES = [tuple(int(v) for v in np.random.default_rng(9000 + i).integers(1, 700, 3)) for i in range(16)]


@pytest.mark.parametrize("m,k,n", _RAND_SHAPES)
def test_seeded_random_shapes_all_forms(ctx, m, k, n):
    """16 seeded random (M, K, N) in [1, 700): every tile edge, K tail and
    scalar/vector load path the planner reaches, all three forms, against
    float64."""
    rng = np.random.default_rng(m * 1_000_003 + k * 1009 + n)
    a = _u(rng, m * k)
    b_nn, b_nt = _u(rng, k * n), _u(rng, n * k)
    a64 = a.reshape(m, k).astype(np.float64)
    cw, fr = _gates(_nn(ctx, a, b_nn, m, n, k), a64, b_nn.reshape(k, n).astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nn", cw, fr)
    cw, fr = _gates(_nt(ctx, a, b_nt, m, n, k), a64, b_nt.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nt", cw, fr)
    x, dy, dest = _u(rng, k * n), _u(rng, k * m), _u(rng, m * n)
    got = _outer(ctx, x, dy, dest, m, n, k)
    cw, fr = _gates(got, dy.reshape(k, m).T.astype(np.float64), x.reshape(k, n).astype(np.float64),
                    dest.reshape(m, n))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("outer", cw, fr)


@pytest.mark.parametrize("cfg", ["256x128:1", "256x128:2", "128x128:1", "128x128:4", "128x64:1",
                                 "128x64:2", "64x64:1", "64x64:4", "64x32:1", "64x32:4", "32x32:1",
                                 "32x32:8", "staged"])
def test_every_tile_config_all_forms(ctx, monkeypatch, cfg):
    """Every kernel variant the planner can pick, forced through the tuning
    override (read on each call), on a whole-tile shape: the 256×128 BK=16
    tile (A k-contiguous forms), the 128×128 / 128×64 / 64×64 / 64×32 / 32×32
    direct-load tiles (the 32-row tiles' k-strided operands swizzled within
    their 32-float rows), split-K 2 to 8 with the ordered reduction, and the
    register-staged kernel.  All three forms against float64."""
    if cfg == "staged":
        monkeypatch.setenv("AUR_GEMM_STAGED", "1")
    else:
        monkeypatch.setenv("AUR_GEMM_CFG", cfg)
    m, k, n = 512, 2048, 384
    rng = np.random.default_rng(7100 + len(cfg))
    a = _u(rng, m * k)
    b_nn, b_nt = _u(rng, k * n), _u(rng, n * k)
    a64 = a.reshape(m, k).astype(np.float64)
    cw, fr = _gates(_nn(ctx, a, b_nn, m, n, k), a64, b_nn.reshape(k, n).astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nn", cfg, cw, fr)
    cw, fr = _gates(_nt(ctx, a, b_nt, m, n, k), a64, b_nt.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nt", cfg, cw, fr)
    x, dy, dest = _u(rng, k * n), _u(rng, k * m), _u(rng, m * n)
    got = _outer(ctx, x, dy, dest, m, n, k)
    cw, fr = _gates(got, dy.reshape(k, m).T.astype(np.float64), x.reshape(k, n).astype(np.float64),
                    dest.reshape(m, n))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("outer", cfg, cw, fr)


@pytest.mark.parametrize("cfg", ["64x32:1", "64x32:2", "32x32:1", "32x32:4"])
def test_small_tiles_ragged_shapes(ctx, monkeypatch, cfg):
    """The 64×32 and 32×32 tiles on a ragged shape (the register-staged
    kernel, partial edge tiles, K not a multiple of 32), all three forms."""
    monkeypatch.setenv("AUR_GEMM_CFG", cfg)
    m, k, n = 100, 300, 70
    rng = np.random.default_rng(7300 + len(cfg))
    a = _u(rng, m * k)
    b_nn, b_nt = _u(rng, k * n), _u(rng, n * k)
    a64 = a.reshape(m, k).astype(np.float64)
    cw, fr = _gates(_nn(ctx, a, b_nn, m, n, k), a64, b_nn.reshape(k, n).astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nn", cfg, cw, fr)
    cw, fr = _gates(_nt(ctx, a, b_nt, m, n, k), a64, b_nt.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nt", cfg, cw, fr)
    x, dy, dest = _u(rng, k * n), _u(rng, k * m), _u(rng, m * n)
    got = _outer(ctx, x, dy, dest, m, n, k)
    cw, fr = _gates(got, dy.reshape(k, m).T.astype(np.float64), x.reshape(k, n).astype(np.float64),
                    dest.reshape(m, n))
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("outer", cfg, cw, fr)


@pytest.mark.parametrize("m,k,n", [(32, 1024, 3072), (32, 1024, 1024), (32, 4096, 1024),
                                   (32, 1024, 8192), (1, 36, 130), (17, 4100, 100), (64, 256, 64),
                                   (48, 2048, 200)])
def test_decode_shaped_nt(ctx, m, k, n):
    """M ≤ 64 A@Bᵀ (the decode projections and head) takes the skinny path:
    with and without a K split, ragged N and M, one-chunk K."""
    rng = np.random.default_rng(6000 + m + k + n)
    a, b = _u(rng, m * k), _u(rng, n * k)
    got = _nt(ctx, a, b, m, n, k)
    cw, fr = _gates(got, a.reshape(m, k).astype(np.float64), b.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)
    again = _nt(ctx, a, b, m, n, k)
    assert np.array_equal(got, again)


def test_k_zero_overwrites_and_accumulate_keeps(ctx):
    from aurora_amd.gpu import GpuBuffer

    c = GpuBuffer.from_slice(ctx, np.full(12, 7.0, np.float32))
    a = GpuBuffer.zeros(ctx, 4)
    ctx.call("aur_gemm_nn", a.ptr, a.ptr, c.ptr, 3, 4, 0)
    assert np.all(c.download() == 0.0)
    c.upload(np.full(12, 7.0, np.float32))
    ctx.call("aur_outer_accum", a.ptr, a.ptr, c.ptr, 3, 4, 0)
    assert np.all(c.download() == 7.0)


def test_strided_gemm_ex_submatrix(ctx):
    """aur_gemm_ex on a sub-block: lda/ldb/ldc larger than the logical width."""
    from aurora_amd.gpu import GpuBuffer

    rng = np.random.default_rng(5)
    M, N, K, lda, ldb, ldc = 96, 80, 72, 100, 84, 92
    A = _u(rng, M * lda)
    B = _u(rng, N * ldb)  # B(k,n) = b[n*ldb + k]  (k-contiguous)
    C0 = _u(rng, M * ldc)
    ab, bb, cb = GpuBuffer.from_slice(ctx, A), GpuBuffer.from_slice(ctx, B), GpuBuffer.from_slice(ctx, C0)
    ctx.call("aur_gemm_ex", 1, 1, ab.ptr, lda, bb.ptr, ldb, cb.ptr, ldc, M, N, K, 1)
    got = cb.download().reshape(M, ldc)
    a64 = A.reshape(M, lda)[:, :K].astype(np.float64)
    b64 = B.reshape(N, ldb)[:, :K].T.astype(np.float64)
    want = C0.reshape(M, ldc).astype(np.float64).copy()
    want[:, :N] += a64 @ b64
    assert np.array_equal(got[:, N:], C0.reshape(M, ldc)[:, N:])  # untouched padding
    assert fro_rel(got[:, :N], want[:, :N]) < TOL_GEMM


# ---- M = B·T = 8192 sweep ------------------------------
SWEEP = [(512, 1536), (512, 512), (512, 2048), (2048, 512)]


@pytest.mark.parametrize("k,n", SWEEP)
def test_config1_sweep_nn_nt(ctx, k, n):
    m = 8192
    rng = np.random.default_rng(10_000 + k + n)
    a = _u(rng, m * k)
    b = _u(rng, k * n)
    a64 = a.reshape(m, k).astype(np.float64)
    b64 = b.reshape(k, n).astype(np.float64)
    cw, fr = _gates(_nn(ctx, a, b, m, n, k), a64, b64)
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nn", cw, fr)
    bt = np.ascontiguousarray(b.reshape(k, n).T).ravel()  # B as [n, k]
    cw, fr = _gates(_nt(ctx, a, bt, m, n, k), a64, b64)
    assert cw < TOL_GEMM and fr < TOL_GEMM, ("nt", cw, fr)


def test_config1_tied_head(ctx):
    m, k, n = 8192, 512, 8192
    rng = np.random.default_rng(10_001)
    h, w_tok = _u(rng, m * k), _u(rng, n * k)
    got = _nt(ctx, h, w_tok, m, n, k)
    cw, fr = _gates(got, h.reshape(m, k).astype(np.float64), w_tok.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)


def test_config1_weight_grad_accumulate(ctx):
    """X[8192,512], dY[8192,2048] summed into an existing dest[2048,512]."""
    t, d_in, d_out = 8192, 512, 2048
    rng = np.random.default_rng(10_002)
    x, dy, dest = _u(rng, t * d_in), _u(rng, t * d_out), _u(rng, d_out * d_in)
    got = _outer(ctx, x, dy, dest, d_out, d_in, t)
    cw, fr = _gates(got, dy.reshape(t, d_out).T.astype(np.float64),
                    x.reshape(t, d_in).astype(np.float64), dest.reshape(d_out, d_in))
    assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)
    # Deterministic: the split-K reduction has a fixed order.
    again = _outer(ctx, x, dy, dest, d_out, d_in, t)
    assert np.array_equal(got, again)


def test_tied_lm_head_gradient_through_both_paths(ctx):
    """tests/gpu_parity.rs:404-467 (tied_lm_head_gradient_matches_cpu_through_both_paths):
    t = 6, d = 16, V = 24.  Logits = h·w_tokᵀ through GemmTransposeBKernel, the
    gradient into h = upstream·w_tok through GemmKernel, both against the CPU
    restatement (tied_lm_head_forward / lm_head_backward, src/transformer/
    embedding.rs:152-206) at the reference's pointwise 5e-2; here also the
    w_tok gradient (upstreamᵀ·h, which the reference test leaves to the CPU)
    through OuterProductAccumKernel into a non-zero gradient, and all three
    against float64 at the GEMM gates."""
    from aurora_amd.gpu import GemmKernel, GemmTransposeBKernel, GpuBuffer, OuterProductAccumKernel

    t, d, v = 6, 16, 24
    rng = np.random.default_rng(0xACE)
    w_tok = (rng.standard_normal(v * d) * 0.02).astype(np.float32)
    h, up = _u(rng, t * d), _u(rng, t * v)
    dw0 = _u(rng, v * d)
    want_logits = oracle.tied_head_forward(h, w_tok, v, d)
    want_dw = dw0.copy()
    want_dh = oracle.lm_head_backward(h, w_tok, up, want_dw, v, d)
    hb, wb, ub = (GpuBuffer.from_slice(ctx, x) for x in (h, w_tok, up))
    logits, dh, dw = GpuBuffer.zeros(ctx, t * v), GpuBuffer.zeros(ctx, t * d), GpuBuffer.from_slice(ctx, dw0)
    GemmTransposeBKernel.new(ctx).dispatch_into(ctx, hb, wb, logits, t, v, d)
    GemmKernel.new(ctx).dispatch_into(ctx, ub, wb, dh, t, d, v)
    OuterProductAccumKernel.new(ctx).dispatch_into(ctx, hb, ub, dw, v, d, t)
    got_logits, got_dh, got_dw = logits.download(), dh.download(), dw.download()
    for x in (hb, wb, ub, logits, dh, dw):
        x.free()
    assert max_rel_err(got_logits, want_logits) < 5e-2
    assert max_rel_err(got_dh, want_dh) < 5e-2
    assert max_rel_err(got_dw, want_dw) < 5e-2
    h64, w64, u64 = (x.astype(np.float64) for x in (h, w_tok, up))
    for got, a64, b64, c0 in ((got_logits, h64.reshape(t, d), w64.reshape(v, d).T, None),
                              (got_dh, u64.reshape(t, v), w64.reshape(v, d), None),
                              (got_dw, u64.reshape(t, v).T, h64.reshape(t, d), dw0.reshape(v, d))):
        cw, fr = _gates(got, a64, b64, c0)
        assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)


def test_nt_equals_nn_on_materialised_transpose(ctx):
    m, k, n = 300, 257, 190
    rng = np.random.default_rng(7)
    a, b = _u(rng, m * k), _u(rng, n * k)
    nt = _nt(ctx, a, b, m, n, k)
    nn = _nn(ctx, a, np.ascontiguousarray(b.reshape(n, k).T).ravel(), m, n, k)
    assert fro_rel(nt, nn) < 1e-6


@pytest.mark.parametrize("form,n,k,cfg,splits", [("nt", 512, 512, "128x128:1", 1), ("nn", 512, 1024, "128x128:1", 1),
                                                ("nt", 1024, 1024, "128x64:1", 1), ("acc", 512, 1024, "128x128:4", 4)])
def test_eight_wave_kernel_bitwise_equals_four_wave(ctx, monkeypatch, form, n, k, cfg, splits):
    """A 128×128 or 128×64 grid of at most one block per CU (split-K
    included) runs 8 waves per block.  Every output is summed in the same
    order as by the 4-wave kernel, so the two agree bit for bit;
    AUR_GEMM_NO_W8 keeps the 4-wave kernel.  m is chosen from the device's
    CU count so that the grid has exactly one block per CU (256 on MI355X)."""
    _, cus = ctx.device_info()
    bn = int(cfg.split("x")[1].split(":")[0])
    col_tiles = n // bn
    if cus % (col_tiles * splits) != 0:
        pytest.skip(f"{cus} CUs: no m gives one {cfg} block per CU at n = {n}")
    m = 128 * (cus // (col_tiles * splits))
    rng = np.random.default_rng(m + n + k)
    monkeypatch.setenv("AUR_GEMM_CFG", cfg)
    if form == "acc":  # dest[m, n] += Σ_t dY[t, m]·X[t, n], t = k
        x, dy, dest = _u(rng, k * n), _u(rng, k * m), _u(rng, m * n)
        run = lambda: _outer(ctx, x, dy, dest, m, n, k)
    else:
        a, b = _u(rng, m * k), _u(rng, k * n)
        run = lambda: (_nt if form == "nt" else _nn)(ctx, a, b, m, n, k)
    eight = run()
    monkeypatch.setenv("AUR_GEMM_NO_W8", "1")
    four = run()
    np.testing.assert_array_equal(eight, four)


def test_split_k_refused_while_captured(ctx, monkeypatch):
    """A split-K GEMM enqueued while the library's stream is being captured
    into a HIP graph, without a caller workspace, is refused (the graph would
    keep the address of the context's grow-only workspace); nothing is
    enqueued, and the same call outside the capture runs."""
    import ctypes

    from aurora_amd._lib import AuroraError, load
    from aurora_amd.gpu import GpuBuffer

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    stream = load().aur_stream(ctx.ptr)
    m, n, k = 128, 128, 4096
    rng = np.random.default_rng(31)
    a, b = _u(rng, m * k), _u(rng, n * k)
    ab, bb, cb = GpuBuffer.from_slice(ctx, a), GpuBuffer.from_slice(ctx, b), GpuBuffer.zeros(ctx, m * n)
    monkeypatch.setenv("AUR_GEMM_CFG", "64x64:4")
    ctx.sync()
    assert hip.hipStreamBeginCapture(stream, 1) == 0  # hipStreamCaptureModeThreadLocal
    try:
        with pytest.raises(AuroraError, match="captured"):
            ctx.call("aur_gemm_nt", ab.ptr, bb.ptr, cb.ptr, m, n, k)
    finally:
        g = ctypes.c_void_p()
        assert hip.hipStreamEndCapture(stream, ctypes.byref(g)) == 0
        if g.value:
            hip.hipGraphDestroy(g)
    ctx.call("aur_gemm_nt", ab.ptr, bb.ptr, cb.ptr, m, n, k)
    got = cb.download()
    for x in (ab, bb, cb):
        x.free()
    cw, fr = _gates(got, a.reshape(m, k).astype(np.float64), b.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)


def test_gemm_ex_rejects_short_leading_dimensions(ctx):
    """aur_gemm_ex refuses a leading dimension shorter than the operand's row
    (lda < k for a k-contiguous A, < m for a k-strided one; likewise ldb with
    k / n; ldc < n) and extents above 2^31 - 1, before anything is launched;
    the same call with the minimal leading dimensions runs."""
    from aurora_amd._lib import AuroraError
    from aurora_amd.gpu import GpuBuffer

    m, n, k = 64, 48, 32
    rng = np.random.default_rng(33)
    a, b = _u(rng, m * k), _u(rng, n * k)
    ab, bb, cb = GpuBuffer.from_slice(ctx, a), GpuBuffer.from_slice(ctx, b), GpuBuffer.zeros(ctx, m * n)
    bad = [(1, 1, k - 4, k, n), (0, 1, m - 4, k, n), (1, 1, k, k - 4, n), (1, 0, k, n - 4, n),
           (1, 1, k, k, n - 4)]
    for ak, bk, lda, ldb, ldc in bad:
        with pytest.raises(AuroraError) as e:
            ctx.call("aur_gemm_ex", ak, bk, ab.ptr, lda, bb.ptr, ldb, cb.ptr, ldc, m, n, k, 0)
        assert e.value.code == 10001 and "leading dimension" in str(e.value), (ak, bk, lda, ldb, ldc)
    with pytest.raises(AuroraError) as e:
        ctx.call("aur_gemm_ex", 1, 1, ab.ptr, 1 << 31, bb.ptr, k, cb.ptr, n, m, n, k, 0)
    assert e.value.code == 10003
    ctx.call("aur_gemm_ex", 1, 1, ab.ptr, k, bb.ptr, k, cb.ptr, n, m, n, k, 0)
    got = cb.download()
    for x in (ab, bb, cb):
        x.free()
    cw, fr = _gates(got, a.reshape(m, k).astype(np.float64), b.reshape(n, k).T.astype(np.float64))
    assert cw < TOL_GEMM and fr < TOL_GEMM, (cw, fr)
