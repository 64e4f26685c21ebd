"""float64 causal attention (forward + gradient) from its definition, used as
the independent high-precision reference for the GPU kernels at sizes where
the fp32 CPU restatement (oracle.mha_heads_*) would be slow.  It is written
from the mathematics (softmax of masked scaled scores; the gradient by the
chain rule), not from the reference's loops.

Layout: q, k, v, d_out are [B, T, H, dh] float64.
"""
import numpy as np


def causal_attention_f64(q, k, v):
    """Returns (out [B,T,H,dh], lse [B,H,T])."""
    B, T, H, dh = q.shape
    scale = 1.0 / np.sqrt(dh)
    out = np.empty_like(q)
    lse = np.empty((B, H, T))
    mask = np.triu(np.ones((T, T), dtype=bool), 1)
    for b in range(B):
        qh = q[b].transpose(1, 0, 2)  # [H,T,dh]
        kh = k[b].transpose(1, 0, 2)
        vh = v[b].transpose(1, 0, 2)
        s = (qh @ kh.transpose(0, 2, 1)) * scale
        s[:, mask] = -np.inf
        m = s.max(-1, keepdims=True)
        e = np.exp(s - m)
        z = e.sum(-1, keepdims=True)
        p = e / z
        out[b] = (p @ vh).transpose(1, 0, 2)
        lse[b] = (m + np.log(z))[..., 0]
    return out, lse


def causal_attention_grad_f64(q, k, v, d_out):
    """Returns (dq, dk, dv) of Σ d_out ⊙ attention(q, k, v)."""
    B, T, H, dh = q.shape
    scale = 1.0 / np.sqrt(dh)
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    mask = np.triu(np.ones((T, T), dtype=bool), 1)
    for b in range(B):
        qh = q[b].transpose(1, 0, 2)
        kh = k[b].transpose(1, 0, 2)
        vh = v[b].transpose(1, 0, 2)
        doh = d_out[b].transpose(1, 0, 2)
        s = (qh @ kh.transpose(0, 2, 1)) * scale
        s[:, mask] = -np.inf
        s -= s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        dvh = p.transpose(0, 2, 1) @ doh
        dp = doh @ vh.transpose(0, 2, 1)
        ds = p * (dp - (p * dp).sum(-1, keepdims=True))
        dqh = (ds @ kh) * scale
        dkh = (ds.transpose(0, 2, 1) @ qh) * scale
        dq[b] = dqh.transpose(1, 0, 2)
        dk[b] = dkh.transpose(1, 0, 2)
        dv[b] = dvh.transpose(1, 0, 2)
    return dq, dk, dv
