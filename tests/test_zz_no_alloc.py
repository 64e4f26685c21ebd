"""aur_outer_accum_noalloc — the allocation-free variant of aur_outer_accum
(split-K partials in the library's per-device scratch array) — against
aur_outer_accum, through the C ABI: two calls in a row, the second smaller,
each bit-identical to the allocating entry point and within the GEMM gate of
a float64 product; a shape whose partials exceed the scratch is refused
before anything runs."""
import numpy as np
import pytest

from tests.parity import componentwise

pytestmark = pytest.mark.gpu


def _case(ctx, rng, d_out, d_in, t):
    from aurora_amd.gpu import GpuBuffer

    x = rng.uniform(-1, 1, (t, d_in)).astype(np.float32)
    dy = rng.uniform(-1, 1, (t, d_out)).astype(np.float32)
    dest0 = rng.uniform(-1, 1, (d_out, d_in)).astype(np.float32)
    bx, bdy = GpuBuffer.from_slice(ctx, x), GpuBuffer.from_slice(ctx, dy)
    ref, got = GpuBuffer.from_slice(ctx, dest0), GpuBuffer.from_slice(ctx, dest0)
    ctx.call("aur_outer_accum", bx.ptr, bdy.ptr, ref.ptr, d_out, d_in, t)
    ctx.call("aur_outer_accum_noalloc", bx.ptr, bdy.ptr, got.ptr, d_out, d_in, t)
    r, g = ref.download().reshape(d_out, d_in), got.download().reshape(d_out, d_in)
    assert np.array_equal(g, r), (d_out, d_in, t, float(np.abs(g - r).max()))
    want = dest0.astype(np.float64) + dy.astype(np.float64).T @ x.astype(np.float64)
    bound = np.abs(dest0).astype(np.float64) + np.abs(dy.astype(np.float64)).T @ np.abs(x.astype(np.float64))
    err = componentwise(g, want, bound)
    assert err < 1e-4, (d_out, d_in, t, err)
    for b in (bx, bdy, ref, got):
        b.free()
    return err


def test_outer_accum_noalloc_matches_outer_accum(ctx):
    rng = np.random.default_rng(21)
    # split-K at both sizes (8 and 4 K ranges of the planner), the second smaller
    e1 = _case(ctx, rng, 1024, 1024, 16384)
    e2 = _case(ctx, rng, 384, 256, 3000)
    print(f"[noalloc] bit-identical to aur_outer_accum; componentwise error vs float64 {e1:.1e}, {e2:.1e}")


def test_outer_accum_noalloc_refuses_oversized_partials(ctx):
    """1536 × 1536 over t = 32768: the planner cuts K into 16 ranges, 37.7 M
    floats of partial tiles > the 16.8 M of scratch."""
    from aurora_amd._lib import AuroraError
    from aurora_amd.gpu import GpuBuffer

    d, t = 1536, 32768
    bx, bdy = GpuBuffer.zeros(ctx, t * d), GpuBuffer.zeros(ctx, t * d)
    dest = GpuBuffer.from_slice(ctx, np.full(d * d, 3.0, np.float32))
    with pytest.raises(AuroraError) as e:
        ctx.call("aur_outer_accum_noalloc", bx.ptr, bdy.ptr, dest.ptr, d, d, t)
    assert e.value.code == 10003
    assert np.all(dest.download() == 3.0)  # nothing ran
    for b in (bx, bdy, dest):
        b.free()


def test_outer_accum_noalloc_replays_from_a_captured_graph(ctx):
    """The callers this entry point is for capture it into a HIP graph: it
    captures (nothing in it allocates, synchronises or clears memory), and
    every replay — with the program's own eager work, a fresh upload of the
    destination and a synchronisation between replays — equals the eager
    aur_outer_accum bit for bit."""
    import ctypes

    from aurora_amd._lib import load
    from aurora_amd.gpu import GpuBuffer

    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    hip.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [vp, vp]
    hip.hipGraphExecDestroy.argtypes = [vp]
    hip.hipGraphDestroy.argtypes = [vp]
    stream = load().aur_stream(ctx.ptr)

    d_out, d_in, t = 512, 384, 8192  # split-K plan: partials in the scratch array
    rng = np.random.default_rng(23)
    x = rng.uniform(-1, 1, (t, d_in)).astype(np.float32)
    dy = rng.uniform(-1, 1, (t, d_out)).astype(np.float32)
    dest0 = rng.uniform(-1, 1, (d_out, d_in)).astype(np.float32)
    bx, bdy = GpuBuffer.from_slice(ctx, x), GpuBuffer.from_slice(ctx, dy)
    ref, got = GpuBuffer.from_slice(ctx, dest0), GpuBuffer.from_slice(ctx, dest0)
    ctx.call("aur_outer_accum", bx.ptr, bdy.ptr, ref.ptr, d_out, d_in, t)
    want = ref.download()

    ctx.sync()
    graph, exe = vp(), vp()
    assert hip.hipStreamBeginCapture(stream, 1) == 0  # hipStreamCaptureModeThreadLocal
    try:
        ctx.call("aur_outer_accum_noalloc", bx.ptr, bdy.ptr, got.ptr, d_out, d_in, t)
    finally:
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
    try:
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for replay in range(3):
            got.upload(dest0)
            # eager work of the program's own between replays
            ctx.call("aur_outer_accum", bx.ptr, bdy.ptr, ref.ptr, d_out, d_in, t)
            ctx.sync()
            assert hip.hipGraphLaunch(exe, stream) == 0
            ctx.sync()
            assert np.array_equal(got.download(), want), replay
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        for b in (bx, bdy, ref, got):
            b.free()
