"""Writes tests/golden/fixtures.npz: inputs and float64 reference outputs of
textbook operations, computed with PyTorch's own CPU routines (independent of
the oracle's C code), used to pin the oracle:

* layer_norm       torch.nn.functional.layer_norm (eps 1e-5) + autograd grads
* gelu_tanh        torch.nn.functional.gelu(approximate="tanh") + its derivative
* cross_entropy    torch.nn.functional.cross_entropy (mean over rows) + grad
* causal_sdpa      torch.nn.functional.scaled_dot_product_attention(is_causal)
                   + autograd dq/dk/dv for a given upstream gradient
* adamw            torch.optim.AdamW, two steps, decay and no-decay groups

and tests/golden/model_fixture.npz: a tiny pre-LN GPT (V 32, d 32, L 2, H 2,
d_ff 64, T 8, B 2, seq_len_max 10) written here from torch primitives alone —
F.embedding + learned positions, F.layer_norm, F.linear for Q/K/V, causal
F.scaled_dot_product_attention, W_o and the residual, LayerNorm 2, fc,
F.gelu(approximate="tanh"), proj and the residual, the final LayerNorm, the
tied head F.linear(h, w_tok) and F.cross_entropy per sequence — following
the reference's block and model (src/transformer/block.rs:157-205,
model.rs:730-788), with the trainer's batch mean (examples/aurora_train.rs:
812-846).  Frozen: logits, per-sequence losses, every parameter gradient
(autograd), one clip + AdamW step with the reference's decay groups
(model.rs:926-1009: w_tok, w_q/k/v/o, w_fc, w_proj decayed; w_pos and every
LayerNorm γ/β not), the AdamW-subset norm of the Muon hybrid (model.rs:
518-560) and one whole Muon hybrid step (model.rs:1023-1107, optimizer.rs:
94-305, restated here in torch float64 matrix algebra).

The reference repository stores no golden vectors (its tests draw inputs at
run time from rand's StdRng), so these library-routine vectors are the
known-answer pins.  Run:  python tests/golden/make_fixtures.py
"""
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "fixtures.npz"
OUT_MODEL = Path(__file__).resolve().parent / "model_fixture.npz"

# The tiny model: vocab, d_model, n_layer, n_head, d_ff, seq_len_max; batch, t.
TINY = dict(vocab=32, d_model=32, n_layer=2, n_head=2, d_ff=64, seq_len_max=10)
TINY_B, TINY_T = 2, 8
LAYER_KEYS = ("ln1_g", "ln1_b", "w_q", "w_k", "w_v", "w_o", "ln2_g", "ln2_b", "w_fc", "w_proj")


def main():
    torch.manual_seed(0)
    rng = np.random.default_rng(1234)
    fx = {}

    # layer norm: 5 rows of 24, random gamma/beta
    x = rng.standard_normal((5, 24)) * 2 + 0.5
    g = rng.standard_normal(24)
    b = rng.standard_normal(24)
    dy = rng.standard_normal((5, 24))
    tx, tg, tb = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, g, b))
    y = torch.nn.functional.layer_norm(tx, (24,), tg, tb, eps=1e-5)
    y.backward(torch.tensor(dy))
    fx.update(ln_x=x, ln_g=g, ln_b=b, ln_dy=dy, ln_y=y.detach().numpy(), ln_dx=tx.grad.numpy(),
              ln_dg=tg.grad.numpy(), ln_db=tb.grad.numpy())

    # gelu (tanh form)
    xg = np.linspace(-6, 6, 97)
    t = torch.tensor(xg, dtype=torch.float64, requires_grad=True)
    yg = torch.nn.functional.gelu(t, approximate="tanh")
    yg.sum().backward()
    fx.update(gelu_x=xg, gelu_y=yg.detach().numpy(), gelu_dy=t.grad.numpy())

    # cross entropy: 7 rows over 33 classes
    logits = rng.standard_normal((7, 33)) * 3
    tgt = rng.integers(0, 33, 7)
    tl = torch.tensor(logits, dtype=torch.float64, requires_grad=True)
    loss = torch.nn.functional.cross_entropy(tl, torch.tensor(tgt), reduction="mean")
    loss.backward()
    fx.update(ce_logits=logits, ce_tgt=tgt.astype(np.uint32), ce_loss=np.array(loss.item()),
              ce_grad=tl.grad.numpy())

    # causal SDPA, 1 head: t = 13, d = 8
    tq, dk = 13, 8
    q, k, v, do = (rng.standard_normal((tq, dk)) for _ in range(4))
    Q, K, Vv = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v))
    o = torch.nn.functional.scaled_dot_product_attention(Q[None, None], K[None, None], Vv[None, None],
                                                         is_causal=True)[0, 0]
    o.backward(torch.tensor(do))
    fx.update(sdpa_q=q, sdpa_k=k, sdpa_v=v, sdpa_do=do, sdpa_o=o.detach().numpy(),
              sdpa_dq=Q.grad.numpy(), sdpa_dk=K.grad.numpy(), sdpa_dv=Vv.grad.numpy())

    # AdamW: two steps, lr 3e-4, betas (0.9, 0.95), eps 1e-8, wd 0.1 on group 0 only
    p0 = rng.standard_normal(11)
    p1 = rng.standard_normal(6)
    g_steps = [(rng.standard_normal(11), rng.standard_normal(6)) for _ in range(2)]
    tp0 = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    tp1 = torch.tensor(p1, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.AdamW([{"params": [tp0], "weight_decay": 0.1},
                             {"params": [tp1], "weight_decay": 0.0}],
                            lr=3e-4, betas=(0.9, 0.95), eps=1e-8)
    outs = []
    for ga, gb in g_steps:
        tp0.grad = torch.tensor(ga, dtype=torch.float64)
        tp1.grad = torch.tensor(gb, dtype=torch.float64)
        opt.step()
        outs.append((tp0.detach().numpy().copy(), tp1.detach().numpy().copy()))
    fx.update(adam_p0=p0, adam_p1=p1, adam_g0_s1=g_steps[0][0], adam_g1_s1=g_steps[0][1],
              adam_g0_s2=g_steps[1][0], adam_g1_s2=g_steps[1][1], adam_p0_s1=outs[0][0],
              adam_p1_s1=outs[0][1], adam_p0_s2=outs[1][0], adam_p1_s2=outs[1][1])

    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({len(fx)} arrays)")
    model_fixture()


def _tiny_params(rng):
    """float32-representable values (the model under test is fp32), drawn
    large enough that every term of the block moves the output: Q/K/V/fc
    weights N(0, 1/d_in), W_o / W_proj likewise, embeddings N(0, 0.5²),
    LayerNorm γ = 1 + N(0, 0.2²), β = N(0, 0.2²)."""
    V, d, L, F, Tm = (TINY[k] for k in ("vocab", "d_model", "n_layer", "d_ff", "seq_len_max"))

    def n(shape, s):
        return (rng.standard_normal(shape) * s).astype(np.float32)

    P = {"w_tok": n((V, d), 0.5), "w_pos": n((Tm, d), 0.5),
         "lnf_g": 1 + n(d, 0.2), "lnf_b": n(d, 0.2)}
    for l in range(L):
        P.update({f"l{l}.ln1_g": 1 + n(d, 0.2), f"l{l}.ln1_b": n(d, 0.2),
                  f"l{l}.w_q": n((d, d), d ** -0.5), f"l{l}.w_k": n((d, d), d ** -0.5),
                  f"l{l}.w_v": n((d, d), d ** -0.5), f"l{l}.w_o": n((d, d), d ** -0.5),
                  f"l{l}.ln2_g": 1 + n(d, 0.2), f"l{l}.ln2_b": n(d, 0.2),
                  f"l{l}.w_fc": n((F, d), d ** -0.5), f"l{l}.w_proj": n((d, F), F ** -0.5)})
    return {k: v.astype(np.float32) for k, v in P.items()}


def _tiny_forward(T, tokens):
    """logits [B, t, V] of the pre-LN GPT from torch primitives."""
    F = torch.nn.functional
    d, H, L = TINY["d_model"], TINY["n_head"], TINY["n_layer"]
    B, t = tokens.shape
    dh = d // H
    h = F.embedding(tokens, T["w_tok"]) + T["w_pos"][:t][None]
    for l in range(L):
        p = lambda k: T[f"l{l}.{k}"]  # noqa: E731
        a = F.layer_norm(h, (d,), p("ln1_g"), p("ln1_b"), eps=1e-5)
        q, k, v = (F.linear(a, p(w)).reshape(B, t, H, dh).transpose(1, 2) for w in ("w_q", "w_k", "w_v"))
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True)  # scale 1/sqrt(dh)
        h = h + F.linear(o.transpose(1, 2).reshape(B, t, d), p("w_o"))
        m = F.layer_norm(h, (d,), p("ln2_g"), p("ln2_b"), eps=1e-5)
        h = h + F.linear(F.gelu(F.linear(m, p("w_fc")), approximate="tanh"), p("w_proj"))
    hf = F.layer_norm(h, (d,), T["lnf_g"], T["lnf_b"], eps=1e-5)
    return F.linear(hf, T["w_tok"])  # tied head


def _decayed(name):
    """model.rs:926-1009: decoupled decay on the matmul weights and w_tok."""
    return name == "w_tok" or name.split(".")[-1] in ("w_q", "w_k", "w_v", "w_o", "w_fc", "w_proj")


def _adamw_subset(name):
    """model.rs:518-560: embeddings, every LayerNorm γ/β and the final LN."""
    return name in ("w_tok", "w_pos", "lnf_g", "lnf_b") or name.split(".")[-1] in (
        "ln1_g", "ln1_b", "ln2_g", "ln2_b")


def _muon_rows_cols(name):
    """Rows × cols the reference passes to muon_apply (model.rs:1076-1081):
    the flat buffer of w_fc ([d_ff, d]) read as d × d_ff, w_proj ([d, d_ff])
    as d_ff × d."""
    d, Ff = TINY["d_model"], TINY["d_ff"]
    return {"w_q": (d, d), "w_k": (d, d), "w_v": (d, d), "w_o": (d, d), "w_fc": (d, Ff),
            "w_proj": (Ff, d)}[name.split(".")[-1]]


def _muon_update(g, mom_buf, rows, cols, momentum=0.95, ns_steps=5):
    """optimizer.rs:238-305 muon_apply's update (Nesterov), float64: returns
    (update scaled by sqrt(max/min), new momentum)."""
    mom_buf = momentum * mom_buf + g
    u = (g + momentum * mom_buf).reshape(rows, cols)
    fro = torch.sqrt((u * u).sum())
    x = u / (fro + 1e-7)
    if rows > cols:
        x = x.T
    a, b, c = 3.4445, -4.7750, 2.0315
    for _ in range(ns_steps):
        A = x @ x.T
        x = a * x + (b * A + c * (A @ A)) @ x
    if rows > cols:
        x = x.T
    return x.reshape(-1) * np.sqrt(max(rows, cols) / min(rows, cols)), mom_buf


def model_fixture():
    rng = np.random.default_rng(20261202)
    P = _tiny_params(rng)
    V, t, B = TINY["vocab"], TINY_T, TINY_B
    tok = rng.integers(0, V, (B, t))
    tgt = rng.integers(0, V, (B, t))
    names = list(P)
    T = {k: torch.tensor(P[k].astype(np.float64), requires_grad=True) for k in names}
    logits = _tiny_forward(T, torch.tensor(tok))
    seq_loss = torch.stack([torch.nn.functional.cross_entropy(logits[b], torch.tensor(tgt[b]))
                            for b in range(B)])
    (seq_loss.sum() / B).backward()  # the CPU trainer: Σ_b grads_b, then × 1/B
    fx = {"tokens": tok.astype(np.uint32), "targets": tgt.astype(np.uint32),
          "cfg": np.array([TINY[k] for k in ("vocab", "d_model", "n_layer", "n_head", "d_ff", "seq_len_max")]),
          "logits": logits.detach().numpy(), "seq_loss": seq_loss.detach().numpy()}
    G = {k: T[k].grad.detach().clone() for k in names}
    for k in names:
        fx[f"p.{k}"] = P[k]
        fx[f"g.{k}"] = G[k].numpy()

    # clip_grads (model.rs:1011-1017: scale by max_norm / norm when above)
    # then step_adamw (lr 3e-4, β 0.9/0.95, eps 1e-8, wd 0.1) through
    # torch.optim.AdamW with the reference's two groups
    norm = float(torch.sqrt(sum((g * g).sum() for g in G.values())))
    max_norm = 0.5 * norm  # the clip is active
    fx.update(grad_norm=np.array(norm), clip_max_norm=np.array(max_norm))
    W = {k: torch.tensor(P[k].astype(np.float64), requires_grad=True) for k in names}
    for k in names:
        W[k].grad = G[k] * (max_norm / norm)
    opt = torch.optim.AdamW([{"params": [W[k] for k in names if _decayed(k)], "weight_decay": 0.1},
                             {"params": [W[k] for k in names if not _decayed(k)], "weight_decay": 0.0}],
                            lr=3e-4, betas=(0.9, 0.95), eps=1e-8)
    opt.step()
    for k in names:
        fx[f"adamw.{k}"] = W[k].detach().numpy()

    # step_muon_hybrid after clip_grads_adamw_subset (model.rs:1101-1107):
    # the subset norm, the subset clipped, AdamW (w_tok decayed only) on the
    # subset, Muon (lr 0.02, momentum 0.95, Nesterov, wd 0, 5 NS steps) on
    # the block matrices from zero momentum — two steps with the same
    # gradients, so the momentum takes part.
    sub = float(torch.sqrt(sum((G[k] * G[k]).sum() for k in names if _adamw_subset(k))))
    sub_max = 0.5 * sub
    fx.update(subset_norm=np.array(sub), subset_max_norm=np.array(sub_max))
    W = {k: torch.tensor(P[k].astype(np.float64), requires_grad=True) for k in names}
    sub_names = [k for k in names if _adamw_subset(k)]
    opt = torch.optim.AdamW([{"params": [W["w_tok"]], "weight_decay": 0.1},
                             {"params": [W[k] for k in sub_names if k != "w_tok"], "weight_decay": 0.0}],
                            lr=6e-4, betas=(0.9, 0.95), eps=1e-8)
    mom = {k: torch.zeros(P[k].size, dtype=torch.float64) for k in names if not _adamw_subset(k)}
    for step in (1, 2):
        for k in sub_names:
            W[k].grad = G[k] * (sub_max / sub)
        opt.step()
        with torch.no_grad():
            for k in mom:
                rows, cols = _muon_rows_cols(k)
                upd, mom[k] = _muon_update(G[k].reshape(-1), mom[k], rows, cols)
                W[k] -= (0.02 * upd).reshape(W[k].shape)
        for k in names:
            fx[f"muon{step}.{k}"] = W[k].detach().numpy().copy()

    np.savez_compressed(OUT_MODEL, **fx)
    print(f"wrote {OUT_MODEL} ({len(fx)} arrays)")


if __name__ == "__main__":
    main()
