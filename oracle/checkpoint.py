"""AURORA05/06/07 checkpoint format restated in numpy — TEST INFRASTRUCTURE ONLY.

Follows src/checkpoint.rs: the layout comment at :9-49, `save` :84-186
(always AURORA07; flags bit i per :70-79; header u32 vocab, d_model,
n_layer, n_head, d_ff, seq_len_max, flags, f32 softcap, u32 canon_kernel
(V6+), u32 sink_tokens (V7+), u32 epoch, u64 step, all little-endian) and
`load` :188-301 (tensors in the order w_tok, w_pos, per block ln1 γ/β,
w_q, w_k, w_v, w_o, ln2 γ/β, w_fc, w_proj, then the final LN γ/β — the
optional-feature tensors only appear when their flag is set, and this
restatement writes them only when asked to, for the refusal tests).

Used by tests/ to write files the GPU model must load and to read what the
GPU model saved; never by the product path.
"""
from __future__ import annotations

import struct

import numpy as np

from oracle.model import Config, tensors

MAGIC = {5: b"AURORA05", 6: b"AURORA06", 7: b"AURORA07"}
FLAG_NAMES = ("rope", "rmsnorm", "relu2", "qk_norm", "untied_head", "swiglu", "layerscale",
              "parallel_block", "diff_attn", "head_bias")


def header_bytes(cfg: Config, epoch: int, step: int, version: int = 7, flags: int = 0,
                 softcap: float = 0.0, canon_kernel: int = 0, sink_tokens: int = 0) -> bytes:
    h = MAGIC[version]
    h += struct.pack("<6I", cfg.vocab, cfg.d_model, cfg.n_layer, cfg.n_head, cfg.d_ff, cfg.seq_len_max)
    h += struct.pack("<If", flags, softcap)
    if version >= 6:
        h += struct.pack("<I", canon_kernel)
    if version >= 7:
        h += struct.pack("<I", sink_tokens)
    h += struct.pack("<IQ", epoch, step)
    return h


def write(path, cfg: Config, P: dict, epoch: int = 0, step: int = 0, version: int = 7, flags: int = 0,
          softcap: float = 0.0, canon_kernel: int = 0, sink_tokens: int = 0) -> None:
    with open(path, "wb") as f:
        f.write(header_bytes(cfg, epoch, step, version, flags, softcap, canon_kernel, sink_tokens))
        for _, _, a in tensors(P):
            f.write(np.ascontiguousarray(a, dtype="<f4").tobytes())


def read(path, cfg: Config | None = None):
    """(header dict, params dict) of a file with every optional feature off."""
    with open(path, "rb") as f:
        data = f.read()
    magic = data[:8]
    version = {v: k for k, v in MAGIC.items()}.get(magic)
    if version is None:
        raise ValueError("bad checkpoint magic")
    vocab, d, n_layer, n_head, d_ff, tmax = struct.unpack_from("<6I", data, 8)
    flags, softcap = struct.unpack_from("<If", data, 32)
    off = 40
    canon = sink = 0
    if version >= 6:
        (canon,) = struct.unpack_from("<I", data, off)
        off += 4
    if version >= 7:
        (sink,) = struct.unpack_from("<I", data, off)
        off += 4
    epoch, step = struct.unpack_from("<IQ", data, off)
    off += 12
    hdr = dict(version=version, vocab=vocab, d_model=d, n_layer=n_layer, n_head=n_head, d_ff=d_ff,
               seq_len_max=tmax, flags=flags, softcap=softcap, canon_kernel=canon, sink_tokens=sink,
               epoch=epoch, step=step, header_len=off)
    c = Config(vocab, d, n_layer, n_head, d_ff, tmax)
    shapes = {"w_tok": (vocab, d), "w_pos": (tmax, d), "lnf_g": (d,), "lnf_b": (d,), "ln1_g": (d,),
              "ln1_b": (d,), "ln2_g": (d,), "ln2_b": (d,), "w_q": (d, d), "w_k": (d, d), "w_v": (d, d),
              "w_o": (d, d), "w_fc": (d_ff, d), "w_proj": (d, d_ff)}

    def take(name):
        nonlocal off
        n = int(np.prod(shapes[name]))
        if off + 4 * n > len(data):
            raise ValueError(f"checkpoint ends inside {name}")
        a = np.frombuffer(data, dtype="<f4", count=n, offset=off).astype(np.float32).reshape(shapes[name])
        off += 4 * n
        return a

    P = {"w_tok": take("w_tok"), "w_pos": take("w_pos"), "layers": []}
    for _ in range(n_layer):
        P["layers"].append({k: take(k) for k in ("ln1_g", "ln1_b", "w_q", "w_k", "w_v", "w_o", "ln2_g",
                                                  "ln2_b", "w_fc", "w_proj")})
    P["lnf_g"], P["lnf_b"] = take("lnf_g"), take("lnf_b")
    hdr["end"] = off
    return hdr, P
