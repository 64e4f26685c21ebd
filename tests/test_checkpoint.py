"""AURORA07 checkpoint I/O (src/checkpoint.rs).

CPU: the format restatement (oracle/checkpoint.py) against the byte layout
documented at checkpoint.rs:9-49, and the C ABI's header reader
(aur_checkpoint_peek needs no GPU) on AURORA05/06/07 files, bad magic,
missing and truncated files.  GPU: the model's save read back by the
restatement, files written by the restatement loaded into the model, the
refusal of optional features this backend lacks, and `load`'s contract of
fresh optimizer moments with the step counter restored (checkpoint.rs:
188-301), checked by one AdamW step against the CPU oracle.
"""
import struct

import numpy as np
import pytest

from oracle import checkpoint as CK
from oracle import model as OM
from tests.parity import fro_rel

C0 = OM.Config(vocab=256, d_model=128, n_layer=2, n_head=4, d_ff=512, seq_len_max=64)
TINY = OM.Config(vocab=16, d_model=8, n_layer=1, n_head=1, d_ff=16, seq_len_max=4)


def _n_params(cfg):
    d = cfg.d_model
    return (cfg.vocab * d + cfg.seq_len_max * d + 2 * d +
            cfg.n_layer * (4 * d + 4 * d * d + 2 * cfg.d_ff * d))


def _random_params(cfg, seed):
    P = OM.init_params(cfg, seed)
    rng = np.random.default_rng(seed + 100)
    for name, l, a in OM.tensors(P):  # non-trivial LN γ/β too
        a[...] = rng.standard_normal(a.shape, dtype=np.float32)
    return P


# ------------------------------------------------------------------ CPU
def test_v7_header_byte_layout():
    """Field offsets of checkpoint.rs:9-31 (V7): magic 0-7, vocab 8, d_model
    12, n_layer 16, n_head 20, d_ff 24, seq_len_max 28, flags 32, softcap 36,
    canon_kernel 40, sink_tokens 44, epoch 48, step 52-59; 60 bytes."""
    h = CK.header_bytes(C0, epoch=7, step=0x0102030405060708, flags=0x200, softcap=30.0,
                        canon_kernel=3, sink_tokens=2)
    assert len(h) == 60
    assert h[:8] == b"AURORA07"
    assert h[8:12] == (256).to_bytes(4, "little") and h[12:16] == (128).to_bytes(4, "little")
    assert h[16:20] == (2).to_bytes(4, "little") and h[20:24] == (4).to_bytes(4, "little")
    assert h[24:28] == (512).to_bytes(4, "little") and h[28:32] == (64).to_bytes(4, "little")
    assert h[32:36] == bytes([0x00, 0x02, 0, 0])
    assert h[36:40] == bytes.fromhex("0000f041")  # 30.0f little-endian
    assert h[40:44] == (3).to_bytes(4, "little") and h[44:48] == (2).to_bytes(4, "little")
    assert h[48:52] == (7).to_bytes(4, "little")
    assert h[52:60] == bytes([8, 7, 6, 5, 4, 3, 2, 1])
    assert len(CK.header_bytes(C0, 0, 0, version=6)) == 56  # no sink_tokens
    assert len(CK.header_bytes(C0, 0, 0, version=5)) == 52  # no canon_kernel either


def test_restatement_roundtrip_and_size(tmp_path):
    P = _random_params(TINY, 1)
    path = tmp_path / "t.ckpt"
    CK.write(path, TINY, P, epoch=2, step=9)
    assert path.stat().st_size == 60 + 4 * _n_params(TINY)
    hdr, Q = CK.read(path)
    assert (hdr["epoch"], hdr["step"], hdr["version"], hdr["end"]) == (2, 9, 7, path.stat().st_size)
    for (_, _, a), (_, _, b) in zip(OM.tensors(P), OM.tensors(Q)):
        np.testing.assert_array_equal(a, b)
    # tensors follow the header in checkpoint order: w_tok first, final β last
    raw = path.read_bytes()
    np.testing.assert_array_equal(np.frombuffer(raw[60:60 + 4 * 16 * 8], "<f4"), P["w_tok"].ravel())
    np.testing.assert_array_equal(np.frombuffer(raw[-32:], "<f4"), P["lnf_b"])


# Every tensor of an AURORA07 file with every optional feature off, in the
# order of the layout comment at checkpoint.rs:27-49 (and `save` :145-186):
# (name, layer, element count).  Written out here, not taken from the
# restatement's own tensor order, so that the two pin each other.
TWO = OM.Config(vocab=12, d_model=16, n_layer=2, n_head=2, d_ff=20, seq_len_max=6)


def _layout_table(cfg):
    d, F = cfg.d_model, cfg.d_ff
    rows = [("w_tok", -1, cfg.vocab * d), ("w_pos", -1, cfg.seq_len_max * d)]
    for l in range(cfg.n_layer):
        rows += [("ln1_g", l, d), ("ln1_b", l, d), ("w_q", l, d * d), ("w_k", l, d * d), ("w_v", l, d * d),
                 ("w_o", l, d * d), ("ln2_g", l, d), ("ln2_b", l, d), ("w_fc", l, F * d), ("w_proj", l, d * F)]
    rows += [("lnf_g", -1, d), ("lnf_b", -1, d)]
    return rows


def _tagged_params(cfg):
    """Each tensor filled with its own index in the table × 1000 + position,
    so any tensor read at another's offset is detected."""
    P = OM.init_params(cfg, 0)
    for i, (name, l, n) in enumerate(_layout_table(cfg)):
        a = P[name] if l < 0 else P["layers"][l][name]
        assert a.size == n, (name, l)
        a[...] = (1000.0 * (i + 1) + np.arange(n, dtype=np.float32)).reshape(a.shape)
    return P


def _check_offsets(raw, cfg):
    off = 60  # the V7 header (test_v7_header_byte_layout)
    for i, (name, l, n) in enumerate(_layout_table(cfg)):
        got = np.frombuffer(raw[off:off + 4 * n], "<f4")
        np.testing.assert_array_equal(got, 1000.0 * (i + 1) + np.arange(n, dtype=np.float32),
                                      err_msg=f"{name}[{l}] at byte {off}")
        off += 4 * n
    assert off == len(raw)


def test_two_layer_tensor_offsets(tmp_path):
    """Byte offset of every per-block tensor of a 2-layer AURORA07 file
    (checkpoint.rs:27-49): the restatement writes each tensor where the
    layout table puts it, and reads each back from there."""
    P = _tagged_params(TWO)
    CK.write(tmp_path / "two.ckpt", TWO, P)
    _check_offsets((tmp_path / "two.ckpt").read_bytes(), TWO)
    # a file assembled byte by byte from the table reads back tensor by tensor
    body = b"".join((1000.0 * (i + 1) + np.arange(n, dtype=np.float32)).astype("<f4").tobytes()
                    for i, (_, _, n) in enumerate(_layout_table(TWO)))
    (tmp_path / "hand.ckpt").write_bytes(CK.header_bytes(TWO, 0, 0) + body)
    _, Q = CK.read(tmp_path / "hand.ckpt")
    for (name, l, a), (_, _, b) in zip(OM.tensors(P), OM.tensors(Q)):
        np.testing.assert_array_equal(a, b, err_msg=f"{name}[{l}]")


@pytest.mark.parametrize("version", [5, 6, 7])
def test_peek_through_c_abi(tmp_path, version):
    from aurora_amd.model import peek_checkpoint

    path = tmp_path / f"v{version}.ckpt"
    CK.write(path, C0, OM.init_params(C0, 0), epoch=4, step=123456789012, version=version, flags=0x12)
    cfg, flags, epoch, step = peek_checkpoint(path)
    assert (cfg.vocab, cfg.d_model, cfg.n_layer, cfg.n_head, cfg.d_ff, cfg.seq_len_max) == \
        (256, 128, 2, 4, 512, 64)
    assert (flags, epoch, step) == (0x12, 4, 123456789012)


def test_peek_errors(tmp_path):
    from aurora_amd._lib import AuroraError
    from aurora_amd.model import peek_checkpoint

    bad = tmp_path / "bad.ckpt"
    bad.write_bytes(b"AURORA99" + bytes(60))
    with pytest.raises(AuroraError) as e:
        peek_checkpoint(bad)
    assert e.value.code == 10001 and "magic" in str(e.value)
    with pytest.raises(AuroraError) as e:
        peek_checkpoint(tmp_path / "missing.ckpt")
    assert e.value.code == 10004
    short = tmp_path / "short.ckpt"
    short.write_bytes(CK.header_bytes(C0, 0, 0)[:40])
    with pytest.raises(AuroraError) as e:
        peek_checkpoint(short)
    assert e.value.code == 10004


# ------------------------------------------------------------------ GPU
def _gpu_model(ctx, cfg, max_batch=8):
    from aurora_amd.model import DecoderTransformerGpu

    return DecoderTransformerGpu(ctx, cfg.vocab, cfg.d_model, cfg.n_layer, cfg.n_head, cfg.d_ff,
                                 cfg.seq_len_max, max_batch)


@pytest.mark.gpu
def test_gpu_save_read_by_restatement(ctx, tmp_path):
    P = _random_params(C0, 2)
    m = _gpu_model(ctx, C0)
    m.load_params(P)
    path = tmp_path / "gpu.ckpt"
    m.save_checkpoint(path, epoch=5, step=77)
    hdr, Q = CK.read(path)
    assert (hdr["version"], hdr["flags"], hdr["softcap"], hdr["epoch"], hdr["step"]) == (7, 0, 0.0, 5, 77)
    assert hdr["end"] == path.stat().st_size == 60 + 4 * _n_params(C0)
    for (name, l, a), (_, _, b) in zip(OM.tensors(P), OM.tensors(Q)):
        np.testing.assert_array_equal(a, b, err_msg=f"{name}[{l}]")
    m.destroy()


@pytest.mark.gpu
def test_gpu_save_two_layer_offsets_and_hand_built_load(ctx, tmp_path):
    """The C++ writer puts every tensor of a 2-layer model at the offset of
    the layout table (checkpoint.rs:27-49), and the C++ reader takes each
    tensor of a file assembled byte by byte from that table."""
    from aurora_amd.model import DecoderTransformerGpu

    P = _tagged_params(TWO)
    m = _gpu_model(ctx, TWO, 1)
    m.load_params(P)
    path = tmp_path / "two_gpu.ckpt"
    m.save_checkpoint(path, epoch=0, step=0)
    _check_offsets(path.read_bytes(), TWO)
    m.destroy()
    hand = tmp_path / "hand.ckpt"
    body = b"".join((1000.0 * (i + 1) + np.arange(n, dtype=np.float32)).astype("<f4").tobytes()
                    for i, (_, _, n) in enumerate(_layout_table(TWO)))
    hand.write_bytes(CK.header_bytes(TWO, 0, 0) + body)
    g = DecoderTransformerGpu.from_checkpoint(ctx, hand, max_batch=1)
    Q = g.read_tensors(grad=False)
    for i, (name, l, n) in enumerate(_layout_table(TWO)):
        got = Q[name] if l < 0 else Q["layers"][l][name]
        np.testing.assert_array_equal(np.ravel(got), 1000.0 * (i + 1) + np.arange(n, dtype=np.float32),
                                      err_msg=f"{name}[{l}]")
    g.destroy()


@pytest.mark.gpu
@pytest.mark.parametrize("version", [5, 7])
def test_gpu_loads_restatement_file(ctx, tmp_path, version):
    from aurora_amd.model import DecoderTransformerGpu

    P = _random_params(C0, 3)
    path = tmp_path / "cpu.ckpt"
    CK.write(path, C0, P, epoch=3, step=17, version=version)
    m = DecoderTransformerGpu.from_checkpoint(ctx, path, max_batch=4)
    Q = m.read_tensors(grad=False)  # flat arrays
    for (name, l, a), (_, _, b) in zip(OM.tensors(P), OM.tensors(Q)):
        np.testing.assert_array_equal(a.ravel(), b, err_msg=f"{name}[{l}]")
    assert m.load_checkpoint(path) == (3, 17)
    m.destroy()


@pytest.mark.gpu
def test_gpu_load_refusals(ctx, tmp_path):
    from aurora_amd._lib import AuroraError

    m = _gpu_model(ctx, C0)
    P = OM.init_params(C0, 0)
    cases = {"rope": dict(flags=1), "untied_head": dict(flags=1 << 4), "softcap": dict(softcap=30.0),
             "sink": dict(sink_tokens=4), "canon": dict(canon_kernel=3)}
    for what, kw in cases.items():
        path = tmp_path / f"{what}.ckpt"
        CK.write(path, C0, P, **kw)
        with pytest.raises(AuroraError) as e:
            m.load_checkpoint(path)
        assert e.value.code == 10003, what
    other = OM.Config(vocab=256, d_model=128, n_layer=3, n_head=4, d_ff=512, seq_len_max=64)
    path = tmp_path / "other.ckpt"
    CK.write(path, other, OM.init_params(other, 0))
    with pytest.raises(AuroraError) as e:
        m.load_checkpoint(path)
    assert e.value.code == 10001
    path = tmp_path / "trunc.ckpt"
    CK.write(path, C0, P)
    path.write_bytes(path.read_bytes()[:-100])
    with pytest.raises(AuroraError) as e:
        m.load_checkpoint(path)
    assert e.value.code == 10004
    m.destroy()


@pytest.mark.gpu
def test_gpu_load_gives_fresh_moments_and_restores_step(ctx, tmp_path):
    """After load, one train step + AdamW equals the CPU oracle's step from
    the checkpoint's parameters with zero moments at t = stored step + 1
    (the bias correction differs clearly from t = 1)."""
    cfg = C0
    rng = np.random.default_rng(5)
    seq = rng.integers(0, cfg.vocab, (8, 65)).astype(np.uint32)
    tok, tgt = seq[:, :64].copy(), seq[:, 1:].copy()
    P = OM.init_params(cfg, 4)
    m = _gpu_model(ctx, cfg)
    m.load_params(P)
    for _ in range(2):  # non-zero moments and step before the load
        m.zero_grad()
        m.train_step_batch(tok, tgt)
        m.step_adamw(lr=3e-4, weight_decay=0.1)
    path = tmp_path / "resume.ckpt"
    CK.write(path, cfg, P, epoch=1, step=5)
    assert m.load_checkpoint(path) == (1, 5)
    m.zero_grad()
    m.train_step_batch(tok, tgt)
    m.step_adamw(lr=3e-4, weight_decay=0.1)
    _, G = OM.batch_grads(P, cfg, tok, tgt)
    st = OM.new_adam_state(P)
    st["step"] = 5
    OM.step_adamw(P, G, st, lr=3e-4, wd=0.1)
    for (name, l, a), (_, _, b) in zip(OM.tensors(m.read_tensors(grad=False)), OM.tensors(P)):
        assert fro_rel(a, b) < 1e-5, (name, l, fro_rel(a, b))
    m.destroy()


@pytest.mark.gpu
def test_gpu_save_load_roundtrip_same_logits(ctx, tmp_path):
    from aurora_amd.model import DecoderTransformerGpu

    P = OM.init_params(C0, 6)
    a = _gpu_model(ctx, C0, 2)
    a.load_params(P)
    path = tmp_path / "rt.ckpt"
    a.save_checkpoint(path, 0, 0)
    b = DecoderTransformerGpu.from_checkpoint(ctx, path, max_batch=2)
    tok = np.random.default_rng(7).integers(0, C0.vocab, (2, 64)).astype(np.uint32)
    np.testing.assert_array_equal(a.forward(tok), b.forward(tok))
    a.destroy()
    b.destroy()
