"""CPU oracle of the reference's model level — TEST INFRASTRUCTURE ONLY.

Composes the C primitives of oracle.c into the reference's pre-LN decoder
(src/transformer/{model,block,attention,ffn,embedding,kv_cache}.rs) with the
optional features off, exactly the configuration the BASELINE configs use:

* forward        model.rs:730-788, block.rs:157-205, transformer/attention.rs:120-200,
                 ffn.rs:91-117, embedding.rs:95-169
* backward       model.rs:796-912 (softmax-CE ×1/T in place, tied head, final LN,
                 blocks reversed, embedding scatter), block.rs:207-283,
                 transformer/attention.rs:221-334, ffn.rs:119-149
* batch step     examples/aurora_train.rs:812-848: per-sequence grads summed in
                 sequence order, scaled by 1/B, then clip + AdamW
* clip / AdamW   model.rs:1011-1017 (L2 over all grads, l2_norm model.rs:442-500),
                 model.rs:926-1009 (decay groups), optimizer.rs:58-90
* KV decode      kv_cache.rs:70-245 (prefill = full forward, generate_step =
                 block_step per layer)

Parameters are a dict of float32 arrays keyed like the C ABI's tensors:
w_tok [V,d], w_pos [Tmax,d], lnf_g, lnf_b, and per layer l a dict with
ln1_g, ln1_b, w_q, w_k, w_v, w_o [d,d], ln2_g, ln2_b, w_fc [d_ff,d],
w_proj [d,d_ff].
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

import oracle as O


@dataclass(frozen=True)
class Config:
    vocab: int
    d_model: int
    n_layer: int
    n_head: int
    d_ff: int
    seq_len_max: int

    @property
    def d_head(self) -> int:
        return self.d_model // self.n_head


LAYER_KEYS = ("ln1_g", "ln1_b", "w_q", "w_k", "w_v", "w_o", "ln2_g", "ln2_b", "w_fc", "w_proj")
DECAY_KEYS = {"w_q", "w_k", "w_v", "w_o", "w_fc", "w_proj"}  # + w_tok (model.rs:931-1007)


def init_params(cfg: Config, seed: int) -> dict:
    """BASELINE init: every weight N(0, 0.02) (nanoGPT), the residual-branch
    outputs W_o and W_proj additionally × 1/sqrt(2·n_layer); LN γ = 1, β = 0.
    (The reference's own init differs — Xavier-uniform Q/K/V/fc, src/attention.rs:171-188,
    zero W_o, src/transformer/attention.rs:59, embeddings U(±0.02·√3),
    src/transformer/embedding.rs:34-43 — parity only needs both sides to start
    from the same tensors.)  Drawn from numpy's PCG64 in a
    fixed order: w_tok, w_pos, then per layer w_q, w_k, w_v, w_o, w_fc, w_proj."""
    rng = np.random.default_rng(seed)
    d, F, V, T = cfg.d_model, cfg.d_ff, cfg.vocab, cfg.seq_len_max
    res = 1.0 / np.sqrt(2.0 * cfg.n_layer)

    def n(*shape, s=0.02):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(s)).astype(np.float32)

    P = {"w_tok": n(V, d), "w_pos": n(T, d),
         "lnf_g": np.ones(d, np.float32), "lnf_b": np.zeros(d, np.float32), "layers": []}
    for _ in range(cfg.n_layer):
        L = {"w_q": n(d, d), "w_k": n(d, d), "w_v": n(d, d), "w_o": n(d, d, s=0.02 * res),
             "w_fc": n(F, d), "w_proj": n(d, F, s=0.02 * res),
             "ln1_g": np.ones(d, np.float32), "ln1_b": np.zeros(d, np.float32),
             "ln2_g": np.ones(d, np.float32), "ln2_b": np.zeros(d, np.float32)}
        P["layers"].append(L)
    return P


def zeros_like(P: dict) -> dict:
    G = {k: np.zeros_like(v) for k, v in P.items() if k != "layers"}
    G["layers"] = [{k: np.zeros_like(v) for k, v in L.items()} for L in P["layers"]]
    return G


def copy_params(P: dict) -> dict:
    Q = {k: v.copy() for k, v in P.items() if k != "layers"}
    Q["layers"] = [{k: v.copy() for k, v in L.items()} for L in P["layers"]]
    return Q


def tensors(P: dict):
    """(name, layer, array) for every tensor, in the l2_norm order of
    model.rs:442-500 (embeddings, then per block LN1, Q, K, V, O, LN2, fc,
    proj, then the final LN)."""
    yield "w_tok", -1, P["w_tok"]
    yield "w_pos", -1, P["w_pos"]
    for l, L in enumerate(P["layers"]):
        for k in ("ln1_g", "ln1_b", "w_q", "w_k", "w_v", "w_o", "ln2_g", "ln2_b", "w_fc", "w_proj"):
            yield k, l, L[k]
    yield "lnf_g", -1, P["lnf_g"]
    yield "lnf_b", -1, P["lnf_b"]


# ----------------------------------------------------------------- forward
def _block_forward(cfg, L, x, t):
    d, H, dh, F = cfg.d_model, cfg.n_head, cfg.d_head, cfg.d_ff
    ln1, c1 = O.layer_norm_forward(L["ln1_g"], L["ln1_b"], x, d)
    q = O.linear_forward(L["w_q"], ln1, d, d)
    k = O.linear_forward(L["w_k"], ln1, d, d)
    v = O.linear_forward(L["w_v"], ln1, d, d)
    heads, probs = O.mha_heads_forward(q, k, v, t, H, dh)
    mha_out = O.linear_forward(L["w_o"], heads, d, d)
    post = (x + mha_out).astype(np.float32)
    ln2, c2 = O.layer_norm_forward(L["ln2_g"], L["ln2_b"], post, d)
    h_pre = O.linear_forward(L["w_fc"], ln2, d, F)
    h_post = O.gelu(h_pre)
    ffn_out = O.linear_forward(L["w_proj"], h_post, F, d)
    z = (post + ffn_out).astype(np.float32)
    cache = dict(x=x, ln1=ln1, c1=c1, q=q, k=k, v=v, heads=heads, probs=probs, post=post, ln2=ln2,
                 c2=c2, h_pre=h_pre, h_post=h_post)
    return z, cache


def forward(P: dict, cfg: Config, tokens):
    """DecoderTransformer::forward for one sequence → (logits [t*V], cache)."""
    tokens = np.asarray(tokens, np.uint32)
    t, d = tokens.size, cfg.d_model
    h = O.embed_forward(P["w_tok"], P["w_pos"], tokens, d)
    blocks = []
    for L in P["layers"]:
        h, c = _block_forward(cfg, L, h, t)
        blocks.append(c)
    h_final, cf = O.layer_norm_forward(P["lnf_g"], P["lnf_b"], h, d)
    logits = O.tied_head_forward(h_final, P["w_tok"], cfg.vocab, d)
    return logits, dict(tokens=tokens, blocks=blocks, h_pre_final=h, cf=cf, h_final=h_final)


# ----------------------------------------------------------------- backward
def _block_backward(cfg, L, G, c, dz, t):
    d, H, dh, F = cfg.d_model, cfg.n_head, cfg.d_head, cfg.d_ff
    # FFN (ffn.rs:119-149)
    d_h_post = O.linear_backward(L["w_proj"], c["h_post"], dz, G["w_proj"], F, d)
    d_h_pre = (d_h_post * O.gelu_backward(c["h_pre"])).astype(np.float32)
    d_ln2 = O.linear_backward(L["w_fc"], c["ln2"], d_h_pre, G["w_fc"], d, F)
    d_ffn_in = O.layer_norm_backward(L["ln2_g"], c["c2"], d_ln2, G["ln2_g"], G["ln2_b"], d)
    d_post = (dz + d_ffn_in).astype(np.float32)
    # MHA (transformer/attention.rs:221-334)
    d_heads = O.linear_backward(L["w_o"], c["heads"], d_post, G["w_o"], d, d)
    dq, dk, dv = O.mha_heads_backward(c["q"], c["k"], c["v"], c["probs"], d_heads, t, H, dh)
    dx_q = O.linear_backward(L["w_q"], c["ln1"], dq, G["w_q"], d, d)
    dx_k = O.linear_backward(L["w_k"], c["ln1"], dk, G["w_k"], d, d)
    dx_v = O.linear_backward(L["w_v"], c["ln1"], dv, G["w_v"], d, d)
    d_ln1 = ((dx_q + dx_k) + dx_v).astype(np.float32)
    d_x_mha = O.layer_norm_backward(L["ln1_g"], c["c1"], d_ln1, G["ln1_g"], G["ln1_b"], d)
    return (d_post + d_x_mha).astype(np.float32)


def backward(P: dict, cfg: Config, cache: dict, logits, targets, G: dict) -> float:
    """DecoderTransformer::backward → mean-over-t loss; grads accumulate into G."""
    targets = np.asarray(targets, np.uint32)
    t, d, V = targets.size, cfg.d_model, cfg.vocab
    total, d_logits = O.softmax_ce(logits, targets, V)
    d_h = O.lm_head_backward(cache["h_final"], P["w_tok"], d_logits, G["w_tok"], V, d)
    dx = O.layer_norm_backward(P["lnf_g"], cache["cf"], d_h, G["lnf_g"], G["lnf_b"], d)
    for l in range(cfg.n_layer - 1, -1, -1):
        dx = _block_backward(cfg, P["layers"][l], G["layers"][l], cache["blocks"][l], dx, t)
    O.embed_backward(cache["tokens"], dx, G["w_tok"], G["w_pos"], d)
    return total / t


def sequence_grads(P: dict, cfg: Config, tokens, targets):
    """Forward + backward of one sequence into fresh grads → (mean NLL, g)."""
    g = zeros_like(P)
    logits, cache = forward(P, cfg, tokens)
    loss = backward(P, cfg, cache, logits, targets, g)
    return loss, g


def batch_grads(P: dict, cfg: Config, tokens, targets, threads: int = 1, reduction: str = "mean"):
    """aurora_train.rs:812-846 without the optimizer: per-sequence grads summed
    in sequence order, then scaled by 1/B ("mean", the CPU trainer) or left
    summed ("sum", the GPU model's train_step_batch, gpu/transformer.rs:
    1555-1559).  Returns (Σ_b loss_b, G).

    threads > 1 computes the sequences concurrently, as the reference's rayon
    par_iter does (aurora_train.rs:828-838); each sequence's arithmetic and
    the in-order sum are unchanged, so the result is bit-identical."""
    tokens = np.asarray(tokens, np.uint32)
    targets = np.asarray(targets, np.uint32)
    B = tokens.shape[0]
    G = zeros_like(P)
    loss = 0.0
    if threads <= 1 or B == 1:
        results = (sequence_grads(P, cfg, tokens[b], targets[b]) for b in range(B))
        for lb, g in results:
            loss += lb
            _add_assign(G, g)
    else:
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(max_workers=min(threads, B)) as ex:
            futs = [ex.submit(sequence_grads, P, cfg, tokens[b], targets[b]) for b in range(B)]
            for f in futs:  # summed in sequence order
                lb, g = f.result()
                loss += lb
                _add_assign(G, g)
                del g
    if reduction == "mean":
        scale_grads(G, 1.0 / B)
    elif reduction != "sum":
        raise ValueError(reduction)
    return loss, G


def _add_assign(G, g):
    for k, v in G.items():
        if k == "layers":
            for Lg, lg in zip(v, g["layers"]):
                for kk in Lg:
                    O.add_assign_(Lg[kk], lg[kk])
        else:
            O.add_assign_(v, g[k])


def scale_grads(G, f: float) -> None:
    for _, _, a in tensors(G):
        O.scale_(a, f)


def l2_norm(G) -> float:
    s = 0.0
    for _, _, a in tensors(G):
        s = O.sumsq_acc(a, s)
    return float(np.sqrt(np.float32(s)))


def clip_grads(G, max_norm: float) -> float:
    n = l2_norm(G)
    if n > max_norm and n > 0.0:
        scale_grads(G, np.float32(max_norm) / np.float32(n))
    return n


def new_adam_state(P):
    return {"step": 0, "m1": zeros_like(P), "m2": zeros_like(P)}


def step_adamw(P, G, state, lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.1) -> None:
    state["step"] += 1
    bc1, bc2 = O.bias_correction(state["step"], beta1, beta2)
    for (name, l, p), (_, _, g), (_, _, m1), (_, _, m2) in zip(
            tensors(P), tensors(G), tensors(state["m1"]), tensors(state["m2"])):
        decay = name == "w_tok" or name in DECAY_KEYS
        O.adamw_apply(p, g, m1, m2, lr, beta1, beta2, eps, wd, bc1, bc2, decay)


# ------------------------------------------------------------ Muon hybrid
MUON_SHAPES = (("w_q", "d", "d"), ("w_k", "d", "d"), ("w_v", "d", "d"), ("w_o", "d", "d"),
               ("w_fc", "d", "F"), ("w_proj", "F", "d"))  # rows × cols as gpu/transformer.rs:858-865 passes them


def new_muon_state(P):
    return [{k: np.zeros_like(L[k]) for k, _, _ in MUON_SHAPES} for L in P["layers"]]


def _adamw_subset(G):
    """The AdamW-managed tensors in model.rs:518-560 order (embeddings, per
    block LN1 γ/β and LN2 γ/β, final LN)."""
    yield "w_tok", -1, G["w_tok"]
    yield "w_pos", -1, G["w_pos"]
    for l, L in enumerate(G["layers"]):
        for k in ("ln1_g", "ln1_b", "ln2_g", "ln2_b"):
            yield k, l, L[k]
    yield "lnf_g", -1, G["lnf_g"]
    yield "lnf_b", -1, G["lnf_b"]


def clip_grads_adamw_subset(G, max_norm: float) -> float:
    """model.rs:1101-1107 with l2_norm_adamw_subset :518-560 (one sequential
    fp32 sum) and scale_adamw_subset :571-..."""
    s = 0.0
    for _, _, g in _adamw_subset(G):
        s = O.sumsq_acc(g, s)
    n = float(np.sqrt(np.float32(s)))
    if n > max_norm and n > 0.0:
        f = np.float32(max_norm) / np.float32(n)
        for _, _, g in _adamw_subset(G):
            O.scale_(g, f)
    return n


def step_muon_hybrid(P, G, adam_state, muon_state, cfg: Config, muon_lr=0.02, momentum=0.95, nesterov=True,
                     muon_wd=0.0, ns_steps=5, lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.1) -> None:
    """model.rs:1023-1090: shared step counter; AdamW on the embeddings (w_tok
    decayed, embed_lr_mult = 1) and LayerNorm γ/β; muon_apply on every block
    matrix with the reference's rows × cols."""
    adam_state["step"] += 1
    bc1, bc2 = O.bias_correction(adam_state["step"], beta1, beta2)
    for (name, l, p), (_, _, g) in zip(_adamw_subset(P), _adamw_subset(G)):
        m1 = adam_state["m1"][name] if l < 0 else adam_state["m1"]["layers"][l][name]
        m2 = adam_state["m2"][name] if l < 0 else adam_state["m2"]["layers"][l][name]
        O.adamw_apply(p, g, m1, m2, lr, beta1, beta2, eps, wd, bc1, bc2, name == "w_tok")
    dims = {"d": cfg.d_model, "F": cfg.d_ff}
    for l, L in enumerate(P["layers"]):
        for k, r, c in MUON_SHAPES:
            O.muon_apply(L[k], G["layers"][l][k], muon_state[l][k], dims[r], dims[c], muon_lr, momentum,
                         nesterov, muon_wd, ns_steps)


# --------------------------------------------------------------- KV decode
class KvCache:
    """KvCache (kv_cache.rs:45-92): per-layer K/V rows of one sequence."""

    def __init__(self, cfg: Config):
        self.cfg = cfg
        self.k = [np.zeros(0, np.float32) for _ in range(cfg.n_layer)]
        self.v = [np.zeros(0, np.float32) for _ in range(cfg.n_layer)]
        self.current_len = 0

    def prefill(self, P, tokens):
        """kv_cache.rs:70-92: full forward, copy each block's K/V; returns the
        forward's logits (the reference returns h_final's last row; callers
        take the first greedy token from the full-forward logits)."""
        logits, cache = forward(P, self.cfg, tokens)
        for l, c in enumerate(cache["blocks"]):
            self.k[l] = c["k"].copy()
            self.v[l] = c["v"].copy()
        self.current_len = len(tokens)
        return logits


def generate_step(P: dict, cfg: Config, kv: KvCache, token: int):
    """kv_cache.rs:97-143 + block_step :147-245 → logits [V]."""
    d, H, dh, F = cfg.d_model, cfg.n_head, cfg.d_head, cfg.d_ff
    pos = kv.current_len
    h = (P["w_tok"][token] + P["w_pos"][pos]).astype(np.float32)
    for l, L in enumerate(P["layers"]):
        ln1, _ = O.layer_norm_forward(L["ln1_g"], L["ln1_b"], h, d)
        q = O.linear_forward(L["w_q"], ln1, d, d)
        k = O.linear_forward(L["w_k"], ln1, d, d)
        v = O.linear_forward(L["w_v"], ln1, d, d)
        kv.k[l] = np.concatenate([kv.k[l].ravel(), k])
        kv.v[l] = np.concatenate([kv.v[l].ravel(), v])
        heads = O.kv_attend(q, kv.k[l], kv.v[l], pos + 1, H, dh)
        post = (h + O.linear_forward(L["w_o"], heads, d, d)).astype(np.float32)
        ln2, _ = O.layer_norm_forward(L["ln2_g"], L["ln2_b"], post, d)
        h_post = O.gelu(O.linear_forward(L["w_fc"], ln2, d, F))
        h = (post + O.linear_forward(L["w_proj"], h_post, F, d)).astype(np.float32)
    hf, _ = O.layer_norm_forward(P["lnf_g"], P["lnf_b"], h, d)
    kv.current_len += 1
    return O.tied_head_forward(hf, P["w_tok"], cfg.vocab, d)


def argmax(logits) -> int:
    """src/transformer/loss.rs argmax: first index of the maximum."""
    return int(np.argmax(np.asarray(logits)))
