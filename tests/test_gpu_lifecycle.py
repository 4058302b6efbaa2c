"""Model lifecycle on the device: the bytes fl_vram_usage reports (GetVRAMUsage,
device.go:159-161; exported by the reference as fletcher_vram_allocated_bytes,
server.go:116-125) come back when a model is freed, and a forward whose
activation buffers cannot be allocated fails cleanly and leaves a model that
reallocates and computes correctly on the next call (the server recovers from
a failed request and keeps serving, embeddings.go:524-536)."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth


def _cfg():
    return synth.nomic(layers=1, vocab_size=2000, max_pos=1024)


def test_vram_usage_returns_after_model_free(ctx, fl):
    cfg = _cfg()
    w = synth.make_weights(cfg)
    lengths = np.array([300, 17, 512], np.int64)
    ids = synth.make_ids(lengths, vocab_lo=200, vocab_hi=2000)
    # A first model creates the context's RoPE tables for these lengths.
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    m.load(w)
    m.forward(ids, lengths)
    m.close()
    before = ctx.vram_usage()[0]
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    m.load(w)
    assert ctx.vram_usage()[0] > before
    m.forward(ids, lengths)
    m.embed(ids, lengths, max_seqs=2, max_tokens=600)
    m.close()
    assert ctx.vram_usage()[0] == before


def test_forward_recovers_after_failed_allocation(ctx, fl):
    cfg = _cfg()
    w = synth.make_weights(cfg)
    lengths = np.array([200, 33], np.int64)
    ids = synth.make_ids(lengths, vocab_lo=200, vocab_hi=2000)
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    try:
        m.load(w)
        want = m.forward(ids, lengths)
        # One sequence of 2^30 tokens: its activations (~1.6 TB for X alone)
        # cannot be allocated, so the call fails before any kernel runs (the
        # device ids are never read).
        d_ids = ctx.int32(ids)
        d_out = ctx.empty((1, cfg.hidden))
        with pytest.raises(fl.FletcherError) as e:
            m.forward_device(d_ids, np.array([1 << 30], np.int64), d_out)
        assert e.value.code == fl.ERR_OOM
        got = m.forward(ids, lengths)
        np.testing.assert_array_equal(got, want)
        d_ids.free()
        d_out.free()
    finally:
        m.close()
