"""Weight layout, folding and rotary tables of the host side, checked against the reference's contract
and the oracle."""

from __future__ import annotations

import torch

from oracle import folded, reference
from turbo_roformer_amd import weights
from turbo_roformer_amd.stack import fold_sublayer, rope_table, sublayer_prefixes

# parameter names of the upstream checkpoints (the list of tests/test_model.py:12-28 in the reference)
UPSTREAM_KEYS = [
    "layers.0.0.layers.0.0.rotary_embed.freqs",
    "layers.0.0.layers.0.0.norm.gamma",
    "layers.0.0.layers.0.0.to_qkv.weight",
    "layers.0.0.layers.0.0.to_gates.weight",
    "layers.0.0.layers.0.0.to_gates.bias",
    "layers.0.0.layers.0.0.to_out.0.weight",
    "layers.0.1.layers.0.1.net.0.gamma",
    "layers.0.1.layers.0.1.net.1.weight",
    "layers.0.1.layers.0.1.net.4.bias",
    "final_norm.gamma",
    "band_split.to_features.0.0.gamma",
    "band_split.to_features.61.1.weight",
    "mask_estimators.0.to_freqs.0.0.0.weight",
    "mask_estimators.0.to_freqs.61.0.2.bias",
]


def test_state_dict_layout_and_count():
    shapes = weights.param_shapes(weights.RESURRECTION_CFG)
    for k in UPSTREAM_KEYS:
        assert k in shapes, k
    assert 50e6 < weights.param_count(weights.RESURRECTION_CFG) < 52e6
    assert len(weights.band_dims(weights.RESURRECTION_CFG)) == 62
    assert sum(weights.DEFAULT_FREQS_PER_BANDS) == 1025


def test_init_is_seeded_and_perturbed():
    a = weights.init_state_dict(weights.TINY_CFG, seed=4)
    b = weights.init_state_dict(weights.TINY_CFG, seed=4)
    c = weights.init_state_dict(weights.TINY_CFG, seed=5)
    assert all(torch.equal(a[k], b[k]) for k in a)
    assert not torch.equal(a["final_norm.gamma"], c["final_norm.gamma"])
    assert a["final_norm.gamma"].std() > 0.1
    w = a["layers.0.0.layers.0.0.to_qkv.weight"]
    assert w.abs().max() <= 1 / 16 + 1e-7  # default Linear bound 1/sqrt(256)
    n = weights.init_state_dict(weights.TINY_CFG, seed=4, init="normal")
    assert abs(float(n["layers.0.0.layers.0.0.to_qkv.weight"].std()) - 0.02) < 1e-3


def test_execution_order():
    sd = weights.init_state_dict(weights.TINY_CFG, seed=0)
    assert sublayer_prefixes(sd) == [
        ("layers.0.0.layers.0", 0), ("layers.0.1.layers.0", 1), ("layers.1.0.layers.0", 0), ("layers.1.1.layers.0", 1),
    ]


def test_fold_matches_oracle_bitwise(tiny_sd):
    ref = folded.fold(tiny_sd, weights.TINY_CFG["depth"])
    for (prefix, mode), P in zip(sublayer_prefixes(tiny_sd), ref):
        w = fold_sublayer(tiny_sd, prefix)
        assert mode == P["mode"]
        assert torch.equal(w["w_qkvg"], P["W"])
        assert torch.equal(w["b_gate"], P["b"][1536:])
        assert torch.equal(w["w_out"], P["Wo"]) and torch.equal(w["w_ff1"], P["W1"])
        assert torch.equal(w["w_ff2"], P["W2"]) and torch.equal(w["b_ff1"], P["b1"]) and torch.equal(w["b_ff2"], P["b2"])


def test_rope_table_matches_oracle_angles():
    f = weights.rotary_freqs()
    for L in (1, 62, 1701):
        t = rope_table(f, L)
        ang = reference.rotary_angles(L, f)
        assert torch.equal(t[0], ang.cos()) and torch.equal(t[1], ang.sin())
