"""CPU oracle for the GEMM / causal-attention hot path — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker (or the timed CPU baseline), never as
the thing shipped: the product (aurora_amd, libaurora_hip.so) has no CPU path.

`oracle.c` restates the reference's Rust CPU functions in C (same loop order
and fp32 summation structure; each function cites the reference file:line).
This module binds it with ctypes and numpy.  `oracle.model` composes those
primitives into the reference's DecoderTransformer forward / backward /
AdamW step and KV-cache decode (src/transformer/*.rs).

Parity status of each function (how it is pinned) is listed in
tests/test_oracle.py; functions without an independent pin would say
"parity unpinned" there.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_P = C.c_void_p
_Z = C.c_size_t
_F = C.c_float
_I = C.c_int

_SIG = {
    "ora_dot": (_F, [_P, _P, _Z]),
    "ora_cpu_gemm": (None, [_P, _P, _P, _Z, _Z, _Z]),
    "ora_cpu_gemm_transpose_b": (None, [_P, _P, _P, _Z, _Z, _Z]),
    "ora_linear_forward": (None, [_P, _P, _P, _Z, _Z, _Z]),
    "ora_linear_forward_seqs": (None, [_P, _P, _P, _Z, _Z, _Z, _Z, _I]),
    "ora_linear_backward": (None, [_P, _P, _P, _P, _P, _Z, _Z, _Z]),
    "ora_outer_accum": (None, [_P, _P, _P, _Z, _Z, _Z]),
    "ora_tied_head_forward": (None, [_P, _P, _P, _Z, _Z, _Z]),
    "ora_lm_head_backward": (None, [_P, _P, _P, _P, _P, _Z, _Z, _Z]),
    "ora_sdpa_forward": (None, [_P, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _I]),
    "ora_sdpa_backward": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _Z, _Z, _Z]),
    "ora_mha_heads_forward": (None, [_P, _P, _P, _P, _P, _P, _Z, _Z, _Z]),
    "ora_mha_heads_backward": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _Z, _Z]),
    "ora_layer_norm_forward": (None, [_P, _P, _F, _P, _P, _P, _P, _P, _Z, _Z]),
    "ora_layer_norm_backward": (None, [_P, _P, _P, _P, _P, _P, _P, _Z, _Z]),
    "ora_gelu": (None, [_P, _P, _Z]),
    "ora_gelu_backward": (None, [_P, _P, _Z]),
    "ora_softmax_ce": (_F, [_P, _P, _P, _Z, _Z]),
    "ora_token_nll": (None, [_P, _P, _P, _Z, _Z]),
    "ora_embed_forward": (None, [_P, _P, _P, _P, _Z, _Z]),
    "ora_embed_backward": (None, [_P, _P, _P, _P, _Z, _Z]),
    "ora_adamw_apply": (None, [_P, _P, _P, _P, _Z, _F, _F, _F, _F, _F, _F, _F, _I]),
    "ora_newton_schulz5": (None, [_P, _Z, _Z, _P, _I]),
    "ora_muon_apply": (None, [_P, _P, _P, _Z, _Z, _F, _F, _I, _F, _I, _P]),
    "ora_bias_correction": (None, [_I, _F, _F, C.POINTER(_F), C.POINTER(_F)]),
    "ora_sumsq_acc": (_F, [_P, _Z, _F]),
    "ora_scale": (None, [_P, _Z, _F]),
    "ora_add_assign": (None, [_P, _P, _Z]),
    "ora_kv_attend": (None, [_P, _P, _P, _P, _P, _Z, _Z, _Z]),
}

_lib = None


def build() -> Path:
    """Compile liboracle.so from oracle.c (make, in-tree)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------------------------------------------------------- GEMMs
def cpu_gemm(a, b, m, k, n) -> np.ndarray:
    """src/gpu/matmul.rs:413 — C[m,n] = A[m,k]·B[k,n]."""
    a, b = f32(a), f32(b)
    c = np.empty(m * n, np.float32)
    lib().ora_cpu_gemm(_p(a), _p(b), _p(c), m, k, n)
    return c


def cpu_gemm_transpose_b(a, b, m, k, n) -> np.ndarray:
    """src/gpu/matmul.rs:429 — C[m,n] = A[m,k]·B[n,k]ᵀ."""
    a, b = f32(a), f32(b)
    c = np.empty(m * n, np.float32)
    lib().ora_cpu_gemm_transpose_b(_p(a), _p(b), _p(c), m, k, n)
    return c


def dot(a, b) -> float:
    a, b = f32(a), f32(b)
    return float(lib().ora_dot(_p(a), _p(b), a.size))


def linear_forward(w, x, d_in, d_out) -> np.ndarray:
    """src/attention.rs:219 — y = x·Wᵀ, W [d_out, d_in]."""
    w, x = f32(w), f32(x)
    t = x.size // d_in
    y = np.empty(t * d_out, np.float32)
    lib().ora_linear_forward(_p(w), _p(x), _p(y), t, d_in, d_out)
    return y


def linear_forward_seqs(w, x, d_in, d_out, rows_per_seq, threads) -> np.ndarray:
    w, x = f32(w), f32(x)
    t = x.size // d_in
    y = np.empty(t * d_out, np.float32)
    lib().ora_linear_forward_seqs(_p(w), _p(x), _p(y), t, rows_per_seq, d_in, d_out, threads)
    return y


def linear_backward(w, x, dy, d_w, d_in, d_out) -> np.ndarray:
    """src/attention.rs:241 — returns dx; d_w (float32, in place) += dyᵀ·x."""
    w, x, dy = f32(w), f32(x), f32(dy)
    assert d_w.dtype == np.float32 and d_w.flags.c_contiguous
    t = x.size // d_in
    dx = np.empty(t * d_in, np.float32)
    lib().ora_linear_backward(_p(w), _p(x), _p(dy), _p(dx), _p(d_w), t, d_in, d_out)
    return dx


def outer_accum(x, d_y, dest, d_out, d_in, t) -> None:
    """src/gpu/reduce.rs:15-115 — dest[d_out,d_in] += Σ_t d_y[t,o]·x[t,i], in place."""
    x, d_y = f32(x), f32(d_y)
    assert dest.dtype == np.float32 and dest.flags.c_contiguous
    lib().ora_outer_accum(_p(x), _p(d_y), _p(dest), d_out, d_in, t)


def tied_head_forward(h, w_tok, vocab, d) -> np.ndarray:
    h, w_tok = f32(h), f32(w_tok)
    t = h.size // d
    out = np.empty(t * vocab, np.float32)
    lib().ora_tied_head_forward(_p(h), _p(w_tok), _p(out), t, vocab, d)
    return out


def lm_head_backward(h, w, d_logits, d_w, vocab, d) -> np.ndarray:
    h, w, d_logits = f32(h), f32(w), f32(d_logits)
    t = h.size // d
    d_h = np.empty(t * d, np.float32)
    lib().ora_lm_head_backward(_p(h), _p(w), _p(d_logits), _p(d_h), _p(d_w), t, vocab, d)
    return d_h


# ------------------------------------------------------------ attention
def sdpa_forward(q, k, v, d_k, d_v, causal=True):
    """src/attention.rs:396 — returns (out [t_q*d_v], probs [t_q*t_k])."""
    q, k, v = f32(q), f32(k), f32(v)
    t_q, t_k = q.size // d_k, k.size // d_k
    out = np.empty(t_q * d_v, np.float32)
    probs = np.empty(t_q * t_k, np.float32)
    lib().ora_sdpa_forward(_p(q), _p(k), _p(v), _p(out), _p(probs), t_q, t_k, d_k, d_v,
                           1 if causal else 0)
    return out, probs


def sdpa_backward(q, k, v, probs, d_out, d_k, d_v):
    """src/attention.rs:474 — returns (dq, dk, dv)."""
    q, k, v, probs, d_out = f32(q), f32(k), f32(v), f32(probs), f32(d_out)
    t_q, t_k = q.size // d_k, k.size // d_k
    dq = np.empty(t_q * d_k, np.float32)
    dk = np.empty(t_k * d_k, np.float32)
    dv = np.empty(t_k * d_v, np.float32)
    s1 = np.empty(t_q * t_k, np.float32)
    s2 = np.empty(t_q * t_k, np.float32)
    lib().ora_sdpa_backward(_p(q), _p(k), _p(v), _p(probs), _p(d_out), _p(dq), _p(dk), _p(dv),
                            _p(s1), _p(s2), t_q, t_k, d_k, d_v)
    return dq, dk, dv


def mha_heads_forward(q, k, v, t, n_head, d_head):
    """src/transformer/attention.rs:142-190 — returns (heads_out [t*d], probs [H*t*t])."""
    q, k, v = f32(q), f32(k), f32(v)
    d = n_head * d_head
    out = np.empty(t * d, np.float32)
    probs = np.empty(n_head * t * t, np.float32)
    scratch = np.empty(4 * t * d_head, np.float32)
    lib().ora_mha_heads_forward(_p(q), _p(k), _p(v), _p(out), _p(probs), _p(scratch), t, n_head,
                                d_head)
    return out, probs


def mha_heads_backward(q, k, v, probs, d_heads_out, t, n_head, d_head):
    """src/transformer/attention.rs:235-300 — returns (dq, dk, dv) each [t*d]."""
    q, k, v, probs, dho = f32(q), f32(k), f32(v), f32(probs), f32(d_heads_out)
    d = n_head * d_head
    dq, dk, dv = (np.empty(t * d, np.float32) for _ in range(3))
    scratch = np.empty(7 * t * d_head + 2 * t * t, np.float32)
    lib().ora_mha_heads_backward(_p(q), _p(k), _p(v), _p(probs), _p(dho), _p(dq), _p(dk), _p(dv),
                                 _p(scratch), t, n_head, d_head)
    return dq, dk, dv


def kv_attend(q_new, k_hist, v_hist, t_total, n_head, d_head) -> np.ndarray:
    """src/transformer/kv_cache.rs:181-219 — one query vs history rows [0, t_total)."""
    q_new, k_hist, v_hist = f32(q_new), f32(k_hist), f32(v_hist)
    out = np.empty(n_head * d_head, np.float32)
    scores = np.empty(max(1, t_total), np.float32)
    lib().ora_kv_attend(_p(q_new), _p(k_hist), _p(v_hist), _p(out), _p(scores), t_total, n_head,
                        d_head)
    return out


# --------------------------------------------------------- step support
def layer_norm_forward(gamma, beta, x, d, eps=1e-5):
    """src/attention.rs:84 — returns (y, cache=(mean, inv_std, x_hat))."""
    gamma, beta, x = f32(gamma), f32(beta), f32(x)
    t = x.size // d
    y = np.empty(t * d, np.float32)
    mean = np.empty(t, np.float32)
    inv_std = np.empty(t, np.float32)
    x_hat = np.empty(t * d, np.float32)
    lib().ora_layer_norm_forward(_p(gamma), _p(beta), eps, _p(x), _p(y), _p(mean), _p(inv_std),
                                 _p(x_hat), t, d)
    return y, (mean, inv_std, x_hat)


def layer_norm_backward(gamma, cache, dy, d_gamma, d_beta, d):
    """src/attention.rs:117 — returns dx; d_gamma/d_beta accumulated in place."""
    gamma, dy = f32(gamma), f32(dy)
    _, inv_std, x_hat = cache
    t = dy.size // d
    dx = np.empty(t * d, np.float32)
    lib().ora_layer_norm_backward(_p(gamma), _p(inv_std), _p(x_hat), _p(dy), _p(dx), _p(d_gamma),
                                  _p(d_beta), t, d)
    return dx


def gelu(x) -> np.ndarray:
    x = f32(x)
    y = np.empty_like(x)
    lib().ora_gelu(_p(x), _p(y), x.size)
    return y


def gelu_backward(x) -> np.ndarray:
    x = f32(x)
    y = np.empty_like(x)
    lib().ora_gelu_backward(_p(x), _p(y), x.size)
    return y


def softmax_ce(logits, targets, v):
    """src/transformer/model.rs:820-858 — returns (Σ_t NLL, d_logits scaled by 1/t)."""
    logits, targets = f32(logits), u32(targets)
    t = targets.size
    d = np.empty(t * v, np.float32)
    total = lib().ora_softmax_ce(_p(logits), _p(targets), _p(d), t, v)
    return float(total), d


def token_nll(logits, targets, v) -> np.ndarray:
    """Per-token NLL [t] without a gradient (src/gpu/softmax_ce.rs:101-102)."""
    logits, targets = f32(logits), u32(targets)
    t = targets.size
    out = np.empty(t, np.float32)
    lib().ora_token_nll(_p(logits), _p(targets), _p(out), t, v)
    return out


def embed_forward(w_tok, w_pos, tokens, d) -> np.ndarray:
    w_tok, w_pos, tokens = f32(w_tok), f32(w_pos), u32(tokens)
    if tokens.size * d > w_pos.size or (tokens.size and int(tokens.max()) * d >= w_tok.size):
        raise ValueError(f"embed_forward: {tokens.size} positions / token ids past the tables")
    out = np.empty(tokens.size * d, np.float32)
    lib().ora_embed_forward(_p(w_tok), _p(w_pos), _p(tokens), _p(out), tokens.size, d)
    return out


def embed_backward(tokens, dy, d_w_tok, d_w_pos, d) -> None:
    tokens, dy = u32(tokens), f32(dy)
    if tokens.size * d > d_w_pos.size or (tokens.size and int(tokens.max()) * d >= d_w_tok.size):
        raise ValueError(f"embed_backward: {tokens.size} positions / token ids past the tables")
    lib().ora_embed_backward(_p(tokens), _p(dy), _p(d_w_tok), _p(d_w_pos), tokens.size, d)


def bias_correction(t, beta1, beta2):
    b1, b2 = C.c_float(), C.c_float()
    lib().ora_bias_correction(t, beta1, beta2, C.byref(b1), C.byref(b2))
    return b1.value, b2.value


def newton_schulz5(g, rows, cols, n_iter=5) -> None:
    """In place on the float32 array g (rows × cols, row-major); optimizer.rs:147-252."""
    m, n = min(rows, cols), max(rows, cols)
    scratch = np.zeros(2 * m * m + 2 * m * n, np.float32)
    lib().ora_newton_schulz5(_p(g), rows, cols, _p(scratch), n_iter)


def muon_apply(params, grads, mom, rows, cols, lr=0.02, momentum=0.95, nesterov=True, wd=0.0,
               ns_steps=5) -> None:
    """optimizer.rs:259-305 on float32 arrays (params and mom updated in place)."""
    m, n = min(rows, cols), max(rows, cols)
    scratch = np.zeros(rows * cols + 2 * m * m + 2 * m * n, np.float32)
    lib().ora_muon_apply(_p(params), _p(grads), _p(mom), rows, cols, lr, momentum, 1 if nesterov else 0,
                         wd, ns_steps, _p(scratch))


def adamw_apply(params, grads, m1, m2, lr, beta1, beta2, eps, wd, bc1, bc2, apply_wd) -> None:
    """src/optimizer.rs:58 — params, m1, m2 updated in place (float32)."""
    grads = f32(grads)
    lib().ora_adamw_apply(_p(params), _p(grads), _p(m1), _p(m2), params.size, lr, beta1, beta2,
                          eps, wd, bc1, bc2, 1 if apply_wd else 0)


def sumsq_acc(x, s: float) -> float:
    x = f32(x)
    return float(lib().ora_sumsq_acc(_p(x), x.size, s))


def scale_(x: np.ndarray, f: float) -> None:
    lib().ora_scale(_p(x), x.size, f)


def add_assign_(dst: np.ndarray, src) -> None:
    src = f32(src)
    lib().ora_add_assign(_p(dst), _p(src), dst.size)
