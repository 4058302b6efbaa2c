"""CPU checks of the weight-file writers in synth.py against the two formats
the reference reads (internal/embeddings/weights/loader.go).

* Raw binary (LoadFromRawBinary, loader.go:29-90): the tensors' float32 values
  back to back in the loader's fixed order.  The order is restated here from
  loader.go:40-88 / :111-148 and the file is cut at the byte offsets it
  implies.
* SafeTensors (LoadFromSafeTensors, loader.go:155-237): the file is read back
  with the `safetensors` library itself, which pins the container format; the
  names are the ones loader.go:199-236 looks up and linear weights are stored
  [out, in] (the HF convention the loader transposes, :209-229).
"""
import sys

import numpy as np
import pytest

synth = sys.modules["longbow_fletcher_amd"].synth


def small_bert():
    return synth.bert_tiny(vocab_size=700, hidden=32, heads=2, intermediate=64, layers=2,
                           max_pos=40)


def small_nomic():
    return synth.nomic(vocab_size=500, hidden=64, heads=2, intermediate=96, layers=1, max_pos=48)


def loader_sequence(cfg):
    """(name here, rows, cols) in LoadFromRawBinary's order: embeddings
    (word, position, token type, LayerNorm gamma/beta), then per layer
    loadSelfAttention (Q, Qb, K, Kb, V, Vb), loadSelfOutput (dense, bias,
    LayerNorm), intermediate dense + bias, output dense + bias + LayerNorm, then
    the pooler dense + bias.  Shapes as NewBertModel allocates them."""
    H, I = cfg.hidden, cfg.intermediate
    Ni = 2 * I if cfg.activation == synth.ACT_SWIGLU else I
    seq = [("word_emb", cfg.vocab_size, H), ("pos_emb", cfg.max_pos, H), ("type_emb", 2, H),
           ("emb_ln_g", 1, H), ("emb_ln_b", 1, H)]
    for l in range(cfg.layers):
        seq += [(f"q_w.{l}", H, H), (f"q_b.{l}", 1, H), (f"k_w.{l}", H, H), (f"k_b.{l}", 1, H),
                (f"v_w.{l}", H, H), (f"v_b.{l}", 1, H),
                (f"o_w.{l}", H, H), (f"o_b.{l}", 1, H), (f"attn_ln_g.{l}", 1, H),
                (f"attn_ln_b.{l}", 1, H),
                (f"inter_w.{l}", H, Ni), (f"inter_b.{l}", 1, Ni),
                (f"out_w.{l}", I, H), (f"out_b.{l}", 1, H), (f"out_ln_g.{l}", 1, H),
                (f"out_ln_b.{l}", 1, H)]
    seq += [("pool_w", H, H), ("pool_b", 1, H)]
    return seq


def nonzero_weights(cfg, seed=5):
    """Seeded weights with every vector non-zero, so a swapped or misplaced
    tensor cannot hide behind zeros/ones."""
    w = synth.make_weights(cfg, seed=seed)
    rng = np.random.default_rng(seed)
    for k in w:
        if w[k].ndim == 1:
            w[k] = rng.standard_normal(w[k].shape).astype(np.float32)
    return w


@pytest.mark.parametrize("make_cfg", [small_bert, small_nomic])
def test_order_matches_loader(make_cfg):
    cfg = make_cfg()
    got = [(name, r, c) for _hf, name, r, c, _b in synth.reference_tensor_order(cfg)]
    assert got == loader_sequence(cfg)


def test_raw_binary_layout(tmp_path):
    cfg = small_bert()
    w = nonzero_weights(cfg)
    path = tmp_path / "w.bin"
    synth.save_raw_binary(cfg, w, path)
    data = np.fromfile(path, dtype="<f4")
    seq = loader_sequence(cfg)
    assert data.size == sum(r * c for _n, r, c in seq)
    off = 0
    for name, r, c in seq:
        np.testing.assert_array_equal(data[off:off + r * c], w[name].reshape(-1), err_msg=name)
        off += r * c


def test_raw_binary_rope_bias_free(tmp_path):
    """Nomic has no position table or biases in use, but the reference file
    still carries them (bert.go allocates them); they are written as zeros."""
    cfg = small_nomic()
    w = nonzero_weights(cfg)
    for k in list(w):
        if "_b." in k and not k.startswith(("attn_ln", "out_ln")):
            del w[k]
    assert "pos_emb" not in w and "q_b.0" not in w
    path = tmp_path / "w.bin"
    synth.save_raw_binary(cfg, w, path)
    data = np.fromfile(path, dtype="<f4")
    off = 0
    for name, r, c in loader_sequence(cfg):
        want = w[name].reshape(-1) if name in w else np.zeros(r * c, np.float32)
        np.testing.assert_array_equal(data[off:off + r * c], want, err_msg=name)
        off += r * c
    assert off == data.size


@pytest.mark.parametrize("make_cfg", [small_bert, small_nomic])
def test_safetensors_read_by_library(tmp_path, make_cfg):
    st = pytest.importorskip("safetensors.numpy")
    cfg = make_cfg()
    w = nonzero_weights(cfg)
    path = tmp_path / "w.safetensors"
    synth.save_safetensors(cfg, w, path)
    got = st.load_file(str(path))
    names = [hf for hf, *_ in synth.reference_tensor_order(cfg)]
    assert sorted(got) == sorted(names)
    assert "encoder.layer.0.attention.self.query.weight" in got
    assert f"encoder.layer.{cfg.layers - 1}.output.LayerNorm.bias" in got
    for hf, name, r, c, _b in synth.reference_tensor_order(cfg):
        a = got[hf]
        assert a.dtype == np.float32
        ref = w[name].reshape(r, c) if name in w else np.zeros((r, c), np.float32)
        if hf.endswith(".weight") and r > 1 and "embeddings" not in hf and "LayerNorm" not in hf:
            assert a.shape == (c, r), hf        # HF [out, in]
            np.testing.assert_array_equal(a.T, ref, err_msg=hf)
        else:
            np.testing.assert_array_equal(a.reshape(r, c), ref, err_msg=hf)
