"""The shared seeded generator: determinism, statistics, framing, ragged lengths."""
import sys

import numpy as np

synth = sys.modules["longbow_fletcher_amd"].synth


def test_splitmix64_known_values():
    # SplitMix64 reference outputs for seed 0 (Vigna's published sequence).
    got = synth.splitmix64(0, 3)
    assert [int(x) for x in got] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_normal_statistics_and_determinism():
    a = synth.normal(1234, 5, 200001, 0.02)
    b = synth.normal(1234, 5, 200001, 0.02)
    np.testing.assert_array_equal(a, b)
    assert abs(float(a.mean())) < 2e-4 and abs(float(a.std()) - 0.02) < 2e-4
    assert not np.array_equal(a[:100], synth.normal(1234, 6, 100, 0.02))


def test_weights_layout_and_inits():
    cfg = synth.nomic(layers=1)
    w = synth.make_weights(cfg)
    assert w["inter_w.0"].shape == (768, 6144)   # fused gate+up (bert.go:770-776)
    assert w["out_w.0"].shape == (3072, 768)
    assert "q_b.0" not in w and "pos_emb" not in w
    assert np.all(w["out_ln_g.0"] == 1) and np.all(w["out_ln_b.0"] == 0)
    tiny = synth.make_weights(synth.bert_tiny())
    assert tiny["pos_emb"].shape == (512, 128) and np.all(tiny["q_b.1"] == 0)


def test_ids_framing_and_range():
    lengths = np.array([2, 10, 128])
    ids = synth.make_ids(lengths)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    assert np.all(ids[starts] == 101) and np.all(ids[starts + lengths - 1] == 102)
    body = np.delete(ids, np.concatenate([starts, starts + lengths - 1]))
    assert body.min() >= 1000 and body.max() < 30000


def test_ragged_lengths():
    L = synth.ragged_lengths(512)
    assert L.min() >= 8 and L.max() <= 512 and len(L) == 512
    assert 40 <= np.median(L) <= 100
    np.testing.assert_array_equal(L, synth.ragged_lengths(512))
