"""Python face of the C ABI, shaped like the reference's `aurora::gpu` surface.

`GpuContext`, `GpuBuffer` and the kernel structs keep the reference's names,
argument order and "caller owns every buffer, dispatch only enqueues"
contract, so parity tests read like the reference's `tests/gpu_parity.rs`:

    ctx = GpuContext.new()
    a = GpuBuffer.from_slice(ctx, a_host); ...
    GemmKernel.new(ctx).dispatch_into(ctx, a, b, c, m, n, k)
    got = c.download(ctx)

Every call goes through libaurora_hip.so; there is no host fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import AuroraError

__all__ = [
    "AuroraError", "GpuContext", "GpuBuffer", "GemmKernel", "GemmTransposeBKernel",
    "OuterProductAccumKernel", "CausalMhaForwardKernel", "CausalMhaBackwardKernel",
    "MhaKvCacheKernel",
]


class GpuContext:
    """One device + one stream (src/gpu/context.rs:5-75)."""

    def __init__(self, ptr: int):
        self.ptr = ptr

    @classmethod
    def new(cls, device: int = 0) -> "GpuContext":
        """GpuContext::new() -> Result (context.rs:22): raises AuroraError."""
        lib = _lib.load()
        out = C.c_void_p()
        rc = lib.aur_init(device, C.byref(out))
        if rc != 0:
            raise AuroraError("aur_init", rc, lib.aur_last_error(None).decode())
        return cls(out.value)

    def call(self, name: str, *args) -> None:
        _lib.call(self.ptr, name, *args)

    def sync(self) -> None:
        self.call("aur_sync")

    def device_info(self) -> tuple[str, int]:
        buf = C.create_string_buffer(256)
        cus = C.c_int()
        self.call("aur_device_info", buf, 256, C.byref(cus))
        return buf.value.decode(), cus.value

    def event(self) -> "GpuEvent":
        return GpuEvent(self)

    def destroy(self) -> None:
        if self.ptr:
            _lib.load().aur_destroy(self.ptr)
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


class GpuEvent:
    """A HIP event recorded on the context's stream (the reference's
    GpuProfiler timestamp marks, src/gpu/profiler.rs:13-138)."""

    def __init__(self, ctx: GpuContext):
        self.ctx = ctx
        out = C.c_void_p()
        ctx.call("aur_event_create", C.byref(out))
        self.ptr = out.value

    def record(self) -> "GpuEvent":
        self.ctx.call("aur_event_record", self.ptr)
        return self

    def elapsed_ms(self, stop: "GpuEvent") -> float:
        ms = C.c_float()
        self.ctx.call("aur_event_elapsed_ms", self.ptr, stop.ptr, C.byref(ms))
        return ms.value

    def destroy(self) -> None:
        if self.ptr:
            self.ctx.call("aur_event_destroy", self.ptr)
            self.ptr = None


class GpuBuffer:
    """Device buffer of `len` elements of `dtype` (src/gpu/buffers.rs:14-192)."""

    def __init__(self, ctx: GpuContext, ptr: int, length: int, dtype=np.float32):
        self.ctx = ctx
        self.ptr = ptr
        self.len = length
        self.dtype = np.dtype(dtype)

    @property
    def nbytes(self) -> int:
        return self.len * self.dtype.itemsize

    @classmethod
    def empty(cls, ctx: GpuContext, length: int, dtype=np.float32) -> "GpuBuffer":
        out = C.c_void_p()
        nbytes = max(1, int(length)) * np.dtype(dtype).itemsize
        ctx.call("aur_malloc", nbytes, C.byref(out))
        return cls(ctx, out.value, int(length), dtype)

    @classmethod
    def zeros(cls, ctx: GpuContext, length: int, dtype=np.float32) -> "GpuBuffer":
        buf = cls.empty(ctx, length, dtype)
        ctx.call("aur_memset0", buf.ptr, buf.nbytes)
        return buf

    @classmethod
    def from_slice(cls, ctx: GpuContext, data) -> "GpuBuffer":
        arr = np.ascontiguousarray(data)
        if arr.dtype == np.float64:
            arr = arr.astype(np.float32)
        buf = cls.empty(ctx, arr.size, arr.dtype)
        buf.upload(arr)
        return buf

    def upload(self, data) -> None:
        arr = np.ascontiguousarray(data, dtype=self.dtype)
        if arr.size > self.len:
            raise ValueError(f"upload of {arr.size} elements into buffer of {self.len}")
        self.ctx.call("aur_h2d", self.ptr, arr.ctypes.data, arr.nbytes)

    def download(self, n: int | None = None) -> np.ndarray:
        n = self.len if n is None else int(n)
        if not 0 <= n <= self.len:
            raise ValueError(f"download of {n} elements from buffer of {self.len}")
        out = np.empty(n, dtype=self.dtype)
        self.ctx.call("aur_d2h", out.ctypes.data, self.ptr, out.nbytes)
        return out

    def zero(self) -> None:
        self.ctx.call("aur_memset0", self.ptr, self.nbytes)

    def free(self) -> None:
        if self.ptr:
            self.ctx.call("aur_free", self.ptr)
            self.ptr = None


def _p(buf) -> int:
    return buf.ptr if isinstance(buf, GpuBuffer) else int(buf)


def _need(what: str, n: int, *bufs) -> None:
    """The kernels touch exactly the extents their dimensions name; a
    GpuBuffer shorter than that is refused before the launch (the reference's
    WGSL had wgpu's bounds-checked buffer access; an out-of-range access on the
    GPU faults).  Raw device pointers carry no length and pass unchecked."""
    for b in bufs:
        if isinstance(b, GpuBuffer) and b.len < n:
            raise ValueError(f"{what}: buffer of {b.len} elements, {n} needed")


class _Kernel:
    @classmethod
    def new(cls, ctx: GpuContext | None = None):
        return cls()


class GemmKernel(_Kernel):
    """C = A·B (src/gpu/matmul.rs:230-356)."""

    def dispatch_into(self, ctx, a, b, c, m, n, k):
        _need("GemmKernel a", m * k, a)
        _need("GemmKernel b", k * n, b)
        _need("GemmKernel c", m * n, c)
        ctx.call("aur_gemm_nn", _p(a), _p(b), _p(c), m, n, k)


class GemmTransposeBKernel(_Kernel):
    """C = A·Bᵀ (src/gpu/matmul.rs:358-409)."""

    def dispatch_into(self, ctx, a, b, c, m, n, k):
        _need("GemmTransposeBKernel a", m * k, a)
        _need("GemmTransposeBKernel b", n * k, b)
        _need("GemmTransposeBKernel c", m * n, c)
        ctx.call("aur_gemm_nt", _p(a), _p(b), _p(c), m, n, k)


class OuterProductAccumKernel(_Kernel):
    """dest[d_out,d_in] += Σ_t d_y[t,d_out]·x[t,d_in] (src/gpu/reduce.rs:125-241)."""

    def dispatch_into(self, ctx, x, d_y, dest, d_out, d_in, t):
        _need("OuterProductAccumKernel x", t * d_in, x)
        _need("OuterProductAccumKernel d_y", t * d_out, d_y)
        _need("OuterProductAccumKernel dest", d_out * d_in, dest)
        ctx.call("aur_outer_accum", _p(x), _p(d_y), _p(dest), d_out, d_in, t)


class CausalMhaForwardKernel(_Kernel):
    """Causal MHA forward (src/gpu/attention.rs:346-483).

    `lse` takes the reference's `probs` slot: [b, n_head, t] row log-sum-exp.
    """

    def dispatch_into(self, ctx, q, k, v, out, lse, t, n_head, d_head, b=1):
        _need("CausalMhaForwardKernel q/k/v/out", b * t * n_head * d_head, q, k, v, out)
        _need("CausalMhaForwardKernel lse", b * n_head * t, lse)
        ctx.call("aur_mha_fwd", _p(q), _p(k), _p(v), _p(out), _p(lse), b, t, n_head, d_head)


class CausalMhaBackwardKernel(_Kernel):
    """Causal MHA backward, dq/dk/dv accumulated (src/gpu/attention.rs:485-801)."""

    @staticmethod
    def workspace_len(t, n_head, b=1) -> int:
        return (_lib.load().aur_mha_bwd_ws_bytes(b, t, n_head) + 3) // 4

    def dispatch_into(self, ctx, q, k, v, out, lse, d_out, dq, dk, dv, ws, t, n_head,
                      d_head, b=1):
        _need("CausalMhaBackwardKernel tensors", b * t * n_head * d_head, q, k, v, out, d_out, dq, dk, dv)
        _need("CausalMhaBackwardKernel lse", b * n_head * t, lse)
        _need("CausalMhaBackwardKernel workspace", self.workspace_len(t, n_head, b), ws)
        ctx.call("aur_mha_bwd", _p(q), _p(k), _p(v), _p(out), _p(lse), _p(d_out), _p(dq),
                 _p(dk), _p(dv), _p(ws), b, t, n_head, d_head)


class MhaKvCacheKernel(_Kernel):
    """Single-query attention against a K/V history (src/gpu/kv_cache.rs:366-466)."""

    @staticmethod
    def scratch_len(n_head, max_len, b=1) -> int:
        return (_lib.load().aur_mha_kv_ws_bytes(b, n_head, max_len) + 3) // 4

    def dispatch_into(self, ctx, q_new, k_history, v_history, out, scratch, t_total, n_head,
                      d_head, max_len):
        _need("MhaKvCacheKernel q_new/out", n_head * d_head, q_new, out)
        _need("MhaKvCacheKernel history", max_len * n_head * d_head, k_history, v_history)
        _need("MhaKvCacheKernel scratch", self.scratch_len(n_head, max_len), scratch)
        ctx.call("aur_mha_kv_step", _p(q_new), _p(k_history), _p(v_history), _p(out),
                 _p(scratch), t_total, n_head, d_head, max_len)

    def dispatch_batched(self, ctx, q_new, k_history, v_history, out, scratch, t_total_dev,
                         t_max, b, n_head, d_head, max_len):
        _need("MhaKvCacheKernel q_new/out", b * n_head * d_head, q_new, out)
        _need("MhaKvCacheKernel history", b * max_len * n_head * d_head, k_history, v_history)
        _need("MhaKvCacheKernel scratch", self.scratch_len(n_head, max_len, b), scratch)
        ctx.call("aur_mha_kv_step_batched", _p(q_new), _p(k_history), _p(v_history),
                 _p(out), _p(scratch), _p(t_total_dev), t_max, b, n_head, d_head, max_len)
