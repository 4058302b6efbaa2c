"""The committed golden fixtures: the oracle reproduces its recorded vectors
(regression), and the generator reproduces the recorded inputs."""
import pathlib
import sys

import numpy as np
import pytest

HERE = pathlib.Path(__file__).parent / "golden"
synth = sys.modules["longbow_fletcher_amd"].synth


@pytest.fixture(scope="module")
def vectors():
    return dict(np.load(HERE / "oracle_vectors.npz"))


@pytest.mark.parametrize("name,cfg,pool", [
    ("bert_tiny", synth.bert_tiny(), 2),
    ("bert_tiny_cls", synth.bert_tiny(), 0),
    ("nomic2", synth.nomic(layers=2), 2),
])
def test_oracle_reproduces_golden(orc, vectors, name, cfg, pool):
    ids, lengths = vectors[f"{name}/ids"], vectors[f"{name}/lengths"]
    np.testing.assert_array_equal(ids, synth.make_ids(lengths, seed=99))
    w = synth.make_weights(cfg, seed=7)
    got = orc.forward(cfg, w, ids, lengths, pool=pool)
    np.testing.assert_allclose(got, vectors[f"{name}/out"], atol=1e-6, rtol=1e-6)
