"""Packed-weight layout, manifest grammar and the synthetic generator (CPU)."""
from __future__ import annotations

import numpy as np
import pytest

from fleet_moe import layout as L
from fleet_moe import synth
from oracle import moe_oracle as orc


def test_moe_layout_offsets_and_alignment():
    lay = L.moe_layout(L.DSV2_LITE, layers=(1, 2))
    ents = list(lay.tensors.values())
    assert [e.name for e in ents] == ["L1.norm_post", "L1.router", "L1.experts", "L1.shared",
                                      "L2.norm_post", "L2.router", "L2.experts", "L2.shared"]
    for a, b in zip(ents, ents[1:]):
        assert b.offset % 256 == 0 and b.offset >= a.offset + a.nbytes
        assert b.offset - (a.offset + a.nbytes) < 256
    assert lay.tensors["L1.experts"].nbytes == 64 * 17_301_504
    assert lay.tensors["L1.shared"].nbytes == 34_603_008
    assert lay.tensors["L1.router"].nbytes == 262_144
    assert L.DSV2_LITE.expert_stride == 8_650_752


def test_manifest_roundtrip_and_grammar():
    lay = L.moe_layout(L.DSV2_LITE, layers=(3,))
    text = lay.manifest()
    lines = text.splitlines()
    assert lines[0].startswith("scalar bytes ")
    assert "scalar rms_eps 1e-06" in lines
    assert "scalar routed_scaling 1.0" in lines
    e = lay.tensors["L3.experts"]
    assert f"tensor L3.experts {e.offset} {e.nbytes}" in lines
    scalars, tensors = L.parse_manifest(text)
    assert scalars["expert_stride"] == 8_650_752 and isinstance(scalars["rms_eps"], float)
    assert tensors["L3.router"] == (lay.tensors["L3.router"].offset, 262_144)
    assert L.dims_from_scalars(scalars) == L.DSV2_LITE
    with pytest.raises(ValueError):
        L.parse_manifest("tensor broken 1\n")


def test_pack_expert_matches_oracle_reader():
    rng = np.random.default_rng(0)
    H, I = 64, 16
    g, u, d = (rng.integers(0, 65535, s).astype(np.uint16) for s in ((I, H), (I, H), (H, I)))
    blk = L.pack_expert(g, u, d)
    assert blk.size == 3 * H * I
    pl = orc.PackedLayer(router=np.zeros(H, np.uint16), experts=np.concatenate([blk, blk]),
                         shared=np.zeros(3 * H * 2 * I, np.uint16), expert_stride=3 * H * I,
                         hidden=H, moe_inter=I)
    gg, uu, dd = pl.expert_f32(1)
    np.testing.assert_array_equal(orc.bf16_bits(gg), g)
    np.testing.assert_array_equal(orc.bf16_bits(uu), u)
    np.testing.assert_array_equal(orc.bf16_bits(dd), d)


def test_synth_keyed_and_deterministic():
    dims = L.MoeDims(hidden=64, moe_inter=16, n_routed=8)
    blob1, lay = synth.moe_layer_blob(seed=5, layer=2, dims=dims, threads=1)
    blob2, _ = synth.moe_layer_blob(seed=5, layer=2, dims=dims, threads=4)
    np.testing.assert_array_equal(blob1, blob2)
    blob3, _ = synth.moe_layer_blob(seed=6, layer=2, dims=dims)
    assert not np.array_equal(blob1, blob3)
    # one expert regenerated alone equals its slice of the blob
    ex = L.view_u16(blob1, lay.tensors["L2.experts"]).reshape(8, dims.expert_stride)
    one = np.zeros(dims.expert_stride, np.uint16)
    synth.fill_expert(one, 5, 2, 3, dims)
    np.testing.assert_array_equal(one, ex[3])
    # norm weight is bf16 1.0
    assert np.all(L.view_u16(blob1, lay.tensors["L2.norm_post"]) == 0x3F80)


def test_synth_statistics():
    w = synth.bf16_to_f32(synth.normal_bf16(0, 1, synth.EXPERT_GATE, 0, (1 << 20,)))
    assert abs(float(w.mean())) < 1e-4
    assert abs(float(w.std()) - 0.02) < 1e-4
    np.testing.assert_array_equal(synth.bf16_bits(w), orc.bf16_bits(w))
    x = synth.hidden_inputs(0, 1000)
    assert x.shape == (1000, 2048) and abs(float(x.std()) - 1) < 1e-2


def test_zipf_bias():
    b = synth.zipf_logit_bias(0)
    p = np.exp(b.astype(np.float64))
    assert abs(p.sum() - 1) < 1e-6
    ranks = np.argsort(-p)
    assert p[ranks[0]] / p[ranks[1]] == pytest.approx(2 ** 1.1, rel=1e-5)
    assert sorted(ranks.tolist()) == list(range(64))
