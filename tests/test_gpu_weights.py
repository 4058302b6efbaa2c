"""GPU checks of the weight-file loaders (fl_model_load_raw,
fl_model_load_safetensors; weights/loader.go:29-90 and :155-237).

A model loaded from a file must produce bit-identical outputs to the same
model given the same weights one tensor at a time (fl_model_set_weight): both
end in the same device buffers.  The SafeTensors file of the second test is
written by the `safetensors` library (HF names, [out, in] linear weights), so
the parser and the transposition are checked against the format's own writer.
Error cases follow loader.go's: missing file, short raw stream, missing
tensor, wrong size, F16 data."""
import json
import struct
import sys
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth
from test_weights_io import nonzero_weights  # noqa: E402


# Real head size (64) and Nomic's width, so loaded weights go through the
# packed layouts of the fast kernels; small vocabularies keep the files small.
def tiny_bert():
    return synth.bert_tiny(vocab_size=2000)


def one_layer_nomic():
    return synth.nomic(vocab_size=2000, layers=1, max_pos=512)


def log(msg):
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)


def forward(fl, ctx, cfg, dtype, load):
    lengths = np.array([7, 1, 23, 12], np.int64)
    ids = synth.make_ids(lengths, vocab_lo=200, vocab_hi=cfg.vocab_size)
    m = fl.Model(ctx, cfg, dtype=dtype, math=fl.MATH_REFERENCE if dtype == fl.F32 else fl.MATH_EXACT)
    try:
        load(m)
        out = m.forward(ids, lengths)
        assert m.status() == (False, False)
        return out
    finally:
        m.close()


def bias_free(cfg, w):
    return {k: v for k, v in w.items() if cfg.has_bias or not (
        "_b." in k and not k.startswith(("attn_ln", "out_ln")))}


@pytest.mark.parametrize("make_cfg,dtype", [(tiny_bert, "F32"), (one_layer_nomic, "F16")])
def test_load_raw_matches_set_weight(ctx, fl, tmp_path, make_cfg, dtype):
    cfg = make_cfg()
    w = bias_free(cfg, nonzero_weights(cfg))
    path = tmp_path / "w.bin"
    synth.save_raw_binary(cfg, w, path)
    log(f"raw {cfg.name} {dtype}")
    dt = getattr(fl, dtype)
    want = forward(fl, ctx, cfg, dt, lambda m: m.load(w))
    got = forward(fl, ctx, cfg, dt, lambda m: m.load_raw(path))
    assert np.isfinite(want).all()
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("make_cfg,dtype", [(tiny_bert, "F32"), (one_layer_nomic, "F16")])
def test_load_safetensors_written_by_library(ctx, fl, tmp_path, make_cfg, dtype):
    st = pytest.importorskip("safetensors.numpy")
    cfg = make_cfg()
    w = bias_free(cfg, nonzero_weights(cfg))
    tensors = {}
    for hf, name, r, c, _b in synth.reference_tensor_order(cfg):
        a = w[name].reshape(r, c) if name in w else np.zeros((r, c), np.float32)
        if hf.endswith(".weight") and r > 1 and "embeddings" not in hf and "LayerNorm" not in hf:
            a = a.T                       # HF linear weights are [out, in]
        elif r == 1:
            a = a.reshape(c)
        tensors[hf] = np.ascontiguousarray(a, np.float32)
    path = tmp_path / "w.safetensors"
    st.save_file(tensors, str(path))
    log(f"safetensors {cfg.name} {dtype}")
    dt = getattr(fl, dtype)
    want = forward(fl, ctx, cfg, dt, lambda m: m.load(w))
    got = forward(fl, ctx, cfg, dt, lambda m: m.load_safetensors(path))
    np.testing.assert_array_equal(got, want)


def _model(fl, ctx, cfg):
    return fl.Model(ctx, cfg, dtype=fl.F32, math=fl.MATH_REFERENCE)


def test_load_errors(ctx, fl, tmp_path):
    st = pytest.importorskip("safetensors.numpy")
    cfg = tiny_bert()
    w = nonzero_weights(cfg)
    m = _model(fl, ctx, cfg)
    try:
        with pytest.raises(fl.FletcherError) as e:
            m.load_raw(tmp_path / "missing.bin")
        assert e.value.code == fl.ERR_IO

        raw = tmp_path / "w.bin"
        synth.save_raw_binary(cfg, w, raw)
        short = tmp_path / "short.bin"
        short.write_bytes(raw.read_bytes()[:-4])
        with pytest.raises(fl.FletcherError) as e:
            m.load_raw(short)
        assert e.value.code == fl.ERR_IO and "pooler.dense.bias" in str(e.value)

        good = tmp_path / "w.safetensors"
        synth.save_safetensors(cfg, w, good)
        full = st.load_file(str(good))

        def variant(fn):
            t = dict(full)
            fn(t)
            p = tmp_path / "v.safetensors"
            st.save_file(t, str(p))
            return p

        name = "encoder.layer.1.intermediate.dense.weight"
        p = variant(lambda t: t.pop(name))
        with pytest.raises(fl.FletcherError) as e:
            m.load_safetensors(p)
        assert e.value.code == fl.ERR_INVALID and name in str(e.value) and "not found" in str(e.value)

        p = variant(lambda t: t.__setitem__(name, t[name][:, :-1].copy()))
        with pytest.raises(fl.FletcherError) as e:
            m.load_safetensors(p)
        assert "size mismatch" in str(e.value)

        p = variant(lambda t: t.__setitem__(name, t[name].astype(np.float16)))
        with pytest.raises(fl.FletcherError) as e:
            m.load_safetensors(p)
        assert e.value.code == fl.ERR_UNSUPPORTED and "F16" in str(e.value)

        # Same element count, reference [in, out] orientation: the transpose check fires.
        p = variant(lambda t: t.__setitem__(name, np.ascontiguousarray(t[name].T)))
        with pytest.raises(fl.FletcherError) as e:
            m.load_safetensors(p)
        assert "shape mismatch for transpose" in str(e.value)

        # Crafted headers whose shape product or data offsets overflow 64 bits
        # are rejected by the checks, not passed through signed overflow.
        def crafted(entry):
            hdr = json.dumps({"embeddings.word_embeddings.weight": entry}).encode()
            p = tmp_path / "crafted.safetensors"
            p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 64)
            return p

        with pytest.raises(fl.FletcherError) as e:
            m.load_safetensors(crafted({"dtype": "F32", "shape": [1 << 62, 4],
                                        "data_offsets": [0, 16]}))
        assert "overflows" in str(e.value)
        want_bytes = cfg.vocab_size * cfg.hidden * 4
        top = (1 << 63) - 1
        with pytest.raises(fl.FletcherError) as e:
            m.load_safetensors(crafted({"dtype": "F32", "shape": [cfg.vocab_size, cfg.hidden],
                                        "data_offsets": [top - want_bytes, top]}))
        assert e.value.code == fl.ERR_IO and "past the end" in str(e.value)
    finally:
        m.close()


def test_bias_free_model_rejects_nonzero_bias(ctx, fl, tmp_path):
    cfg = one_layer_nomic()
    w = nonzero_weights(cfg)
    w["k_b.0"] = np.full(cfg.hidden, 0.5, np.float32)
    path = tmp_path / "w.bin"
    synth.save_raw_binary(cfg, w, path)
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    try:
        with pytest.raises(fl.FletcherError) as e:
            m.load_raw(path)
        assert e.value.code == fl.ERR_INVALID and "attention.self.key.bias" in str(e.value)
    finally:
        m.close()
