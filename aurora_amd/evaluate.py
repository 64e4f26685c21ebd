"""Overlapping-window validation scoring over DecoderTransformerGpu.eval_step_batch.

Mirrors the reference's GPU evaluation caller (examples/aurora_train.rs:1665-1686
eval_windows / cap_windows, :1733-1765 evaluate_gpu; bits_per_byte from
src/text_io.rs:43-48): windows of seq_len start every seq_len/2 tokens; the
first window is scored from position 0, every later one only on its last
seq_len - stride positions, so each validation token is scored once with at
least stride tokens of left context.  Windows go to the device in batches of
the model's max_batch, one eval_step_batch call (one forward, one NLL
download) per batch.
"""
from __future__ import annotations

import math

import numpy as np

LN_2 = np.float32(math.log(2.0))


def eval_windows(val_len: int, seq_len: int) -> tuple[list[int], int]:
    """(window starts, scored tail) — examples/aurora_train.rs:1665-1674."""
    stride = max(seq_len // 2, 1)
    starts = []
    p = 0
    while p + seq_len + 1 < val_len:
        starts.append(p)
        p += stride
    return starts, seq_len - stride


def cap_windows(starts: list[int], cap: int) -> list[int]:
    """Even subsample to at most cap starts, keeping start 0; cap 0 keeps all
    (examples/aurora_train.rs:1680-1686)."""
    if cap == 0 or len(starts) <= cap:
        return starts
    step = len(starts) // cap
    return starts[::step][:cap]


def bits_per_byte(total_nats: float, n_bytes: int) -> float:
    """src/text_io.rs:43-48, in f32 like the reference."""
    if n_bytes == 0:
        return 0.0
    return float(np.float32(total_nats) / np.float32(n_bytes) / LN_2)


def evaluate_gpu(model, val_toks, seq_len: int, comp: float, max_windows: int = 0) -> float:
    """Validation bits per byte of val_toks (examples/aurora_train.rs:1733-1765).

    comp is the bytes-per-token compression ratio the caller measured; the
    token count is scaled by it (truncated) before the division, like the
    reference.  Returns +inf when val_toks holds no complete window.
    """
    val = np.ascontiguousarray(val_toks, dtype=np.uint32).ravel()
    if val.size <= seq_len + 1:
        return math.inf
    starts, scored_tail = eval_windows(val.size, seq_len)
    starts = cap_windows(starts, max_windows)
    total_nats = np.float32(0.0)
    total_tokens = 0
    for ci in range(0, len(starts), model.max_batch):
        chunk = starts[ci:ci + model.max_batch]
        inputs = np.stack([val[p:p + seq_len] for p in chunk])
        targets = np.stack([val[p + 1:p + seq_len + 1] for p in chunk])
        nlls = model.eval_step_batch(inputs, targets)
        for wi in range(len(chunk)):
            scored_from = 0 if (ci == 0 and wi == 0) else scored_tail
            win = np.float32(0.0)
            for x in nlls[wi * seq_len + scored_from:(wi + 1) * seq_len]:
                win = np.float32(win + x)
            total_nats = np.float32(total_nats + win)
            total_tokens += seq_len - scored_from
    return bits_per_byte(float(total_nats), int(np.float32(total_tokens) * np.float32(comp)))
