"""Writes tests/golden/fixtures.npz: inputs and float64 reference outputs of
textbook operations, computed with PyTorch's own CPU routines (independent of
the oracle's C code), used to pin the oracle:

* layer_norm       torch.nn.functional.layer_norm (eps 1e-5) + autograd grads
* gelu_tanh        torch.nn.functional.gelu(approximate="tanh") + its derivative
* cross_entropy    torch.nn.functional.cross_entropy (mean over rows) + grad
* causal_sdpa      torch.nn.functional.scaled_dot_product_attention(is_causal)
                   + autograd dq/dk/dv for a given upstream gradient
* adamw            torch.optim.AdamW, two steps, decay and no-decay groups

The reference repository stores no golden vectors (its tests draw inputs at
run time from rand's StdRng), so these library-routine vectors are the
known-answer pins.  Run:  python tests/golden/make_fixtures.py
"""
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "fixtures.npz"


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


if __name__ == "__main__":
    main()
