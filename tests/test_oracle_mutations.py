"""The model-level pins of tests/test_oracle.py catch wiring mistakes.

Each case plants one plausible mistake in an in-memory copy of
oracle/model.py (the file itself is untouched) — LayerNorm 2 fed from the
block input instead of the post-attention residual, the final LayerNorm's
γ and β swapped, K and V projections swapped, w_pos put in the decayed
AdamW group, w_fc / w_proj given the other rows × cols in Muon, the LN2
parameters left out of the Muon hybrid's AdamW subset — and runs the
fixture comparisons against the copy: each mistake must fail at least one
of them.  CPU only.
"""
import sys
import types
from pathlib import Path

import pytest

from oracle import model as OM
from tests import test_oracle as T

SRC = (Path(OM.__file__)).read_text()

MUTATIONS = {
    "ln2_from_block_input": ('ln2, c2 = O.layer_norm_forward(L["ln2_g"], L["ln2_b"], post, d)',
                             'ln2, c2 = O.layer_norm_forward(L["ln2_g"], L["ln2_b"], x, d)'),
    "final_ln_gamma_beta_swapped": ('h_final, cf = O.layer_norm_forward(P["lnf_g"], P["lnf_b"], h, d)',
                                    'h_final, cf = O.layer_norm_forward(P["lnf_b"], P["lnf_g"], h, d)'),
    "k_v_swapped": ('    k = O.linear_forward(L["w_k"], ln1, d, d)\n    v = O.linear_forward(L["w_v"], ln1, d, d)\n'
                    '    heads',
                    '    k = O.linear_forward(L["w_v"], ln1, d, d)\n    v = O.linear_forward(L["w_k"], ln1, d, d)\n'
                    '    heads'),
    "w_pos_decayed": ('decay = name == "w_tok" or name in DECAY_KEYS',
                      'decay = name in ("w_tok", "w_pos") or name in DECAY_KEYS'),
    "muon_ffn_orientation": ('("w_fc", "d", "F"), ("w_proj", "F", "d")', '("w_fc", "F", "d"), ("w_proj", "d", "F")'),
    "ln2_out_of_adamw_subset": ('for k in ("ln1_g", "ln1_b", "ln2_g", "ln2_b"):\n            yield k, l, L[k]',
                                'for k in ("ln1_g", "ln1_b"):\n            yield k, l, L[k]'),
}

CHECKS = ("test_model_forward_matches_torch_definition", "test_model_batch_grads_match_torch_autograd",
          "test_clip_and_adamw_match_torch_with_reference_decay_groups",
          "test_muon_hybrid_matches_torch_definition")


def _mutant(old: str, new: str) -> types.ModuleType:
    assert SRC.count(old) == 1, old
    name = "oracle_model_mutant"
    mod = types.ModuleType(name)
    mod.__dict__["__file__"] = OM.__file__
    sys.modules[name] = mod  # dataclasses resolve their module through sys.modules
    try:
        exec(compile(SRC.replace(old, new), "oracle/model.py (mutant)", "exec"), mod.__dict__)
    finally:
        del sys.modules[name]
    return mod


def _failures(mod, monkeypatch) -> list[str]:
    monkeypatch.setattr(T, "OM", mod)
    failed = []
    for name in CHECKS:
        try:
            getattr(T, name)()
        except AssertionError:
            failed.append(name)
    return failed


def test_unmutated_copy_passes(monkeypatch):
    old = MUTATIONS["w_pos_decayed"][0]
    assert _failures(_mutant(old, old), monkeypatch) == []


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistake_is_caught(name, monkeypatch):
    assert _failures(_mutant(*MUTATIONS[name]), monkeypatch), f"{name} went unnoticed"
