"""Python face of the model-level C ABI (aur_model_*, aur_kv_cache_*):
DecoderTransformerGpu and KvCacheGpu, with the reference's method names
(src/gpu/transformer.rs, src/gpu/kv_cache.rs).  Every call runs on the
device through libaurora_hip.so."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .gpu import GpuContext

LAYER_TENSORS = ("ln1_g", "ln1_b", "w_q", "w_k", "w_v", "w_o", "ln2_g", "ln2_b", "w_fc", "w_proj")
GLOBAL_TENSORS = ("w_tok", "w_pos", "lnf_g", "lnf_b")


class ModelConfig(C.Structure):
    """aur_model_config (TransformerConfig, src/transformer/model.rs:24-127)."""
    _fields_ = [("vocab", C.c_uint32), ("d_model", C.c_uint32), ("n_layer", C.c_uint32),
                ("n_head", C.c_uint32), ("d_ff", C.c_uint32), ("seq_len_max", C.c_uint32)]


def peek_checkpoint(path):
    """Header of an AURORA05/06/07 file: (ModelConfig, flags, epoch, step)."""
    lib = _lib.load()
    cfg, flags, epoch, step = ModelConfig(), C.c_uint32(), C.c_uint32(), C.c_uint64()
    rc = lib.aur_checkpoint_peek(str(path).encode(), C.byref(cfg), C.byref(flags), C.byref(epoch),
                                 C.byref(step))
    if rc != 0:
        raise _lib.AuroraError("aur_checkpoint_peek", rc, lib.aur_last_error(None).decode())
    return cfg, flags.value, epoch.value, step.value


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


class DecoderTransformerGpu:
    def __init__(self, ctx: GpuContext, vocab, d_model, n_layer, n_head, d_ff, seq_len_max,
                 max_batch: int):
        self.ctx = ctx
        self.cfg = ModelConfig(vocab, d_model, n_layer, n_head, d_ff, seq_len_max)
        out = C.c_void_p()
        ctx.call("aur_model_create", C.byref(self.cfg), max_batch, C.byref(out))
        self.ptr = out.value
        self.max_batch = max_batch

    def _call(self, name, *args):
        lib = _lib.load()
        rc = getattr(lib, name)(self.ptr, *args)
        if rc != 0:
            raise _lib.AuroraError(name, rc, lib.aur_last_error(self.ctx.ptr).decode())

    def tensor_ptr(self, name: str, layer: int = -1, grad: bool = False) -> tuple[int, int]:
        p, n = C.c_void_p(), C.c_size_t()
        self._call("aur_model_tensor", name.encode(), layer, 1 if grad else 0, C.byref(p), C.byref(n))
        return p.value, n.value

    def get(self, name: str, layer: int = -1, grad: bool = False) -> np.ndarray:
        p, n = self.tensor_ptr(name, layer, grad)
        out = np.empty(n, np.float32)
        self.ctx.call("aur_d2h", out.ctypes.data, p, out.nbytes)
        return out

    def set(self, name: str, data, layer: int = -1) -> None:
        p, n = self.tensor_ptr(name, layer)
        arr = np.ascontiguousarray(data, dtype=np.float32).ravel()
        if arr.size != n:
            raise ValueError(f"{name}[{layer}]: {arr.size} values for a tensor of {n}")
        self.ctx.call("aur_h2d", p, arr.ctypes.data, arr.nbytes)

    def load_params(self, P: dict) -> None:
        """Upload a parameter dict (oracle.model layout)."""
        for k in GLOBAL_TENSORS:
            self.set(k, P[k])
        for l, L in enumerate(P["layers"]):
            for k in LAYER_TENSORS:
                self.set(k, L[k], l)

    def read_tensors(self, grad: bool) -> dict:
        """Parameters (grad=False) or gradients (grad=True) in the same dict layout."""
        P = {k: self.get(k, -1, grad) for k in GLOBAL_TENSORS}
        P["layers"] = [{k: self.get(k, l, grad) for k in LAYER_TENSORS}
                       for l in range(self.cfg.n_layer)]
        return P

    def zero_grad(self) -> None:
        self._call("aur_model_zero_grad")

    def step_muon_hybrid(self, muon_lr=0.02, momentum=0.95, nesterov=True, muon_wd=0.0, ns_steps=5,
                         lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1) -> None:
        """step_muon_hybrid (model.rs:1023): Muon on the Q/K/V/O/fc/proj
        matrices, AdamW on embeddings and LayerNorm γ/β."""
        self._call("aur_model_step_muon_hybrid", muon_lr, momentum, 1 if nesterov else 0, muon_wd,
                   ns_steps, lr, beta1, beta2, eps, weight_decay)

    def clip_grads_adamw_subset(self, max_norm: float, want_norm: bool = True) -> float:
        n = C.c_float(float("nan"))
        self._call("aur_model_clip_grads_adamw_subset", max_norm, C.byref(n) if want_norm else None)
        return n.value

    # ---- AURORA07 checkpoints (src/checkpoint.rs) ----
    def save_checkpoint(self, path, epoch: int = 0, step: int = 0) -> None:
        """checkpoint::save: AURORA07, every optional feature off."""
        self._call("aur_model_save_checkpoint", str(path).encode(), epoch, step)

    def load_checkpoint(self, path) -> tuple[int, int]:
        """checkpoint::load into this model (same dimensions): parameters,
        fresh optimizer moments, optimizer step = the stored step.
        Returns (epoch, step)."""
        e, st = C.c_uint32(), C.c_uint64()
        self._call("aur_model_load_checkpoint", str(path).encode(), C.byref(e), C.byref(st))
        return e.value, st.value

    @classmethod
    def from_checkpoint(cls, ctx: GpuContext, path, max_batch: int):
        """A model sized from the checkpoint's header, then loaded from it."""
        cfg, flags, epoch, step = peek_checkpoint(path)
        m = cls(ctx, cfg.vocab, cfg.d_model, cfg.n_layer, cfg.n_head, cfg.d_ff, cfg.seq_len_max, max_batch)
        m.load_checkpoint(path)
        return m

    def train_step_batch(self, tokens, targets, reduction: str = "mean") -> float:
        """Forward + CE + backward of b sequences; grads accumulate, combined
        over the batch as their mean ("mean", the CPU trainer) or their sum
        ("sum", src/gpu/transformer.rs:1555-1559).  Returns Σ_b mean_t NLL."""
        red = {"mean": 0, "sum": 1}[reduction]
        tok, tgt = _u32(tokens), _u32(targets)
        b, t = tok.shape
        loss = C.c_float()
        self._call("aur_model_train_step_batch_ex", tok.ctypes.data, tgt.ctypes.data, b, t, red,
                   C.byref(loss))
        return loss.value

    def train_step(self, tokens, targets) -> float:
        """Single sequence (src/gpu/transformer.rs:1535): mean-over-t loss."""
        return self.train_step_batch(np.asarray(tokens)[None, :], np.asarray(targets)[None, :], "sum")

    def grad_norm(self) -> float:
        n = C.c_float()
        self._call("aur_model_grad_norm", C.byref(n))
        return n.value

    # ---- state snapshot (src/gpu/transformer.rs:1152-1240) ----
    def state_bytes(self) -> int:
        n = C.c_size_t()
        self._call("aur_model_state_bytes", C.byref(n))
        return n.value

    def snapshot_state(self):
        """A device buffer holding the parameters and optimizer state (its .step
        attribute the optimizer step), copied on the device."""
        from .gpu import GpuBuffer
        buf = GpuBuffer.empty(self.ctx, self.state_bytes() // 4)
        self.refresh_state(buf)
        return buf

    def refresh_state(self, buf) -> None:
        st = C.c_uint64()
        self._call("aur_model_state_save", buf.ptr, buf.nbytes, C.byref(st))
        buf.step = st.value

    def restore_state(self, buf) -> None:
        self._call("aur_model_state_load", buf.ptr, buf.nbytes, buf.step)

    def forward(self, tokens, want_logits: bool = True):
        tok = _u32(tokens)
        b, t = tok.shape
        out = np.empty((b * t, self.cfg.vocab), np.float32) if want_logits else None
        self._call("aur_model_forward", tok.ctypes.data, b, t, out.ctypes.data if want_logits else None)
        return out

    def eval_step_batch(self, inputs, targets) -> np.ndarray:
        """Per-token NLL (nats) of b equal-length windows, flat [b·t]
        window-major; the caller slices per window
        (src/gpu/transformer.rs:1734-1775).  No gradient or optimizer state
        is touched."""
        if len(inputs) != len(targets):
            raise ValueError("eval_step_batch: inputs and targets differ in window count")
        if len(inputs) == 0:
            return np.empty(0, np.float32)
        tok, tgt = _u32(inputs), _u32(targets)
        if tok.ndim != 2 or tok.shape != tgt.shape:
            raise ValueError("eval_step_batch: windows must all have one length, targets the same shape")
        b, t = tok.shape
        out = np.empty(b * t, np.float32)
        self._call("aur_model_eval_step_batch", tok.ctypes.data, tgt.ctypes.data, b, t, out.ctypes.data)
        return out

    def eval_step_per_token(self, tokens, targets) -> np.ndarray:
        """Per-position NLL of one window (src/gpu/transformer.rs:1779-1811)."""
        return self.eval_step_batch([tokens], [targets])

    def eval_step(self, tokens, targets) -> float:
        """Sum of the window's per-token NLL (src/gpu/transformer.rs:1723-1725);
        summed in f32 in position order like the reference's iterator sum."""
        s = np.float32(0.0)
        for x in self.eval_step_per_token(tokens, targets):
            s = np.float32(s + x)
        return float(s)

    def clip_grads(self, max_norm: float, want_norm: bool = True) -> float:
        n = C.c_float(float("nan"))
        self._call("aur_model_clip_grads", max_norm, C.byref(n) if want_norm else None)
        return n.value

    def step_adamw(self, lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1) -> None:
        self._call("aur_model_step_adamw", lr, beta1, beta2, eps, weight_decay)

    def clip_step_adamw(self, max_norm, lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8,
                        weight_decay=0.1) -> float:
        n = C.c_float()
        self._call("aur_model_clip_step_adamw", max_norm, lr, beta1, beta2, eps, weight_decay,
                   C.byref(n))
        return n.value

    # KV decode
    def kv_cache(self, batch: int, max_len: int) -> "KvCacheGpu":
        return KvCacheGpu(self, batch, max_len)

    def prefill_kv(self, cache: "KvCacheGpu", tokens) -> np.ndarray:
        tok = _u32(tokens)
        b, t = tok.shape
        out = np.empty((b, self.cfg.vocab), np.float32)
        self._call("aur_model_prefill_kv", cache.ptr, tok.ctypes.data, b, t, out.ctypes.data)
        return out

    def generate_step_kv(self, cache: "KvCacheGpu", tokens=None, want_logits=True):
        """One decode step for every sequence; tokens=None feeds the previous argmax.
        Returns (logits [b, V] or None, argmax tokens [b])."""
        b = cache.batch
        tok = _u32(tokens) if tokens is not None else None
        logits = np.empty((b, self.cfg.vocab), np.float32) if want_logits else None
        nxt = np.empty(b, np.uint32)
        self._call("aur_model_generate_step", cache.ptr, tok.ctypes.data if tok is not None else None,
                   logits.ctypes.data if want_logits else None, nxt.ctypes.data)
        return logits, nxt

    def generate_greedy(self, cache: "KvCacheGpu", n_steps: int, collect: bool = True):
        out = np.empty((n_steps, cache.batch), np.uint32) if collect else None
        self._call("aur_model_generate_greedy", cache.ptr, n_steps,
                   out.ctypes.data if collect else None)
        return out

    def destroy(self) -> None:
        if self.ptr:
            _lib.load().aur_model_destroy(self.ptr)
            self.ptr = None


class KvCacheGpu:
    def __init__(self, model: DecoderTransformerGpu, batch: int, max_len: int):
        self.model = model
        self.batch = batch
        self.max_len = max_len
        out = C.c_void_p()
        model._call("aur_kv_cache_create", batch, max_len, C.byref(out))
        self.ptr = out.value

    @property
    def current_len(self) -> int:
        n = C.c_uint32()
        rc = _lib.load().aur_kv_cache_len(self.ptr, C.byref(n))
        if rc:
            raise _lib.AuroraError("aur_kv_cache_len", rc, "")
        return n.value

    def reset(self) -> None:
        rc = _lib.load().aur_kv_cache_reset(self.ptr)
        if rc:
            raise _lib.AuroraError("aur_kv_cache_reset", rc, "")

    def history(self, layer: int) -> tuple[np.ndarray, np.ndarray]:
        k, v = C.c_void_p(), C.c_void_p()
        rc = _lib.load().aur_kv_cache_history(self.ptr, layer, C.byref(k), C.byref(v))
        if rc:
            raise _lib.AuroraError("aur_kv_cache_history", rc, "")
        n = self.batch * self.max_len * self.model.cfg.d_model
        out = []
        for p in (k.value, v.value):
            a = np.empty(n, np.float32)
            self.model.ctx.call("aur_d2h", a.ctypes.data, p, a.nbytes)
            out.append(a.reshape(self.batch, self.max_len, -1))
        return out[0], out[1]

    def destroy(self) -> None:
        if self.ptr:
            _lib.load().aur_kv_cache_destroy(self.ptr)
            self.ptr = None
