"""GPU checks of fl_model_embed, the token-budget batching loop of
runInferenceOnDevice (internal/embeddings/embeddings.go:690-775) with copies
overlapped on their own streams.

* The batch plan is the reference loop's, restated here from
  embeddings.go:704-731 (a batch ends before the sequence that would pass
  max_seqs sequences or max_tokens tokens; a longer sequence runs alone).
* Every batch's outputs equal a plain fl_model_forward of that batch, bit for
  bit; and every sequence's output equals a one-batch forward of all
  sequences to 1e-6 (sequences are computed independently, so batch
  composition only moves rows).
* A sample is checked against the CPU oracle at the fp16 bar.
* The per-batch NaN flag (embeddings.go:757-764) marks exactly the sequences
  of the batch whose output holds a NaN, also where several batches of the
  plan run as one forward, and fl_model_status reports the plan's last batch.
"""
import sys
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth


def log(msg):
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)


def reference_plan(lengths, max_seqs, max_tokens):
    plan, i, n = [], 0, len(lengths)
    while i < n:
        size, tokens = 0, 0
        for j in range(i, n):
            if size >= max_seqs:
                break
            if tokens + lengths[j] > max_tokens and size > 0:
                break
            tokens += int(lengths[j])
            size += 1
        if size == 0:
            size = 1
        plan.append((i, size))
        i += size
    return plan


@pytest.fixture(scope="module")
def nomic_model(fl, ctx):
    cfg = synth.nomic(layers=2)
    w = synth.make_weights(cfg)
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    m.load(w)
    yield cfg, w, m
    m.close()


@pytest.mark.parametrize("max_seqs,max_tokens", [(64, 4096), (512, 16384), (1, 16384), (512, 100)])
def test_embed_matches_batched_forward(nomic_model, max_seqs, max_tokens):
    cfg, _w, m = nomic_model
    lengths = synth.ragged_lengths(300, seed=11)
    lengths[7] = 512                       # longer than max_tokens=100: runs alone
    ids = synth.make_ids(lengths, seed=12)
    log(f"embed max_seqs={max_seqs} max_tokens={max_tokens} T={lengths.sum()}")
    out, nan, nb = m.embed(ids, lengths, max_seqs=max_seqs, max_tokens=max_tokens)
    plan = reference_plan(lengths, max_seqs, max_tokens)
    assert nb == len(plan)
    assert not nan.any()
    starts = np.concatenate([[0], np.cumsum(lengths)])
    for first, count in plan[:6] + plan[-3:]:
        bid = ids[starts[first]:starts[first + count]]
        want = m.forward(bid, lengths[first:first + count])
        np.testing.assert_array_equal(out[first:first + count], want)
    whole = m.forward(ids, lengths)
    np.testing.assert_allclose(out, whole, rtol=0, atol=1e-6)


def test_embed_oracle_sample(nomic_model, orc):
    cfg, w, m = nomic_model
    lengths = synth.ragged_lengths(96, seed=21)
    ids = synth.make_ids(lengths, seed=22)
    out, _nan, nb = m.embed(ids, lengths, max_seqs=512, max_tokens=2048)
    assert nb > 1
    rows = [0, 13, 50, int(np.argmax(lengths)), 95]
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    sub = np.concatenate([ids[starts[r]:starts[r] + lengths[r]] for r in rows])
    orc.set_threads(8)
    want = orc.forward(cfg, w, sub, lengths[rows])
    got = out[rows].astype(np.float64)
    cos = (got * want).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))
    log(f"embed vs oracle min cos {cos.min():.6f}")
    assert cos.min() >= 0.999


def test_fp16_output_is_rne_of_fp32(nomic_model, fl):
    """The fp16 transport (processOutput's Cast(Float16) + ExtractBytes,
    embeddings.go:256-286): fl_model_forward_ex / fl_model_embed_ex with
    FL_F16 deliver exactly numpy's round-to-nearest-even of the fp32 vectors."""
    cfg, _w, m = nomic_model
    lengths = synth.ragged_lengths(70, seed=31)
    ids = synth.make_ids(lengths, seed=32)
    f32 = m.forward(ids, lengths)
    f16 = m.forward(ids, lengths, out_dtype=fl.F16)
    assert f16.dtype == np.float16
    np.testing.assert_array_equal(f16.view(np.uint16), f32.astype(np.float16).view(np.uint16))
    e32, _n, nb = m.embed(ids, lengths, max_seqs=16, max_tokens=2048)
    e16, _n, nb16 = m.embed(ids, lengths, max_seqs=16, max_tokens=2048, out_dtype=fl.F16)
    assert nb16 == nb > 2
    np.testing.assert_array_equal(e16.view(np.uint16), e32.astype(np.float16).view(np.uint16))
    with pytest.raises(fl.FletcherError):
        m.forward(ids, lengths, out_dtype=fl.BF16)


def test_embed_edge_cases(nomic_model):
    cfg, _w, m = nomic_model
    out, nan, nb = m.embed(np.zeros(0, np.int64), np.zeros(0, np.int64))
    assert out.shape == (0, cfg.hidden) and nb == 0
    lengths = np.array([3], np.int64)
    ids = synth.make_ids(lengths)
    out, nan, nb = m.embed(ids, lengths, max_seqs=0, max_tokens=0)  # reference: one sequence per batch
    assert nb == 1
    np.testing.assert_array_equal(out, m.forward(ids, lengths))
    bad = ids.copy()
    bad[1] = cfg.vocab_size
    with pytest.raises(Exception):
        m.embed(bad, lengths)


def test_embed_nan_flag_per_batch(fl, ctx):
    cfg = synth.nomic(layers=1)
    w = synth.make_weights(cfg)
    w["word_emb"] = w["word_emb"].copy()
    w["word_emb"][777] = np.nan
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    try:
        m.load(w)
        lengths = np.full(12, 40, np.int64)
        ids = synth.make_ids(lengths, seed=3)
        ids[5 * 40 + 7] = 777                 # sequence 5, in batch 1 of 4-sequence batches
        out, nan, nb = m.embed(ids, lengths, max_seqs=4, max_tokens=16384)
        assert nb == 3
        assert nan.tolist() == [False] * 4 + [True] * 4 + [False] * 4
        assert np.isnan(out[5]).any() and np.isfinite(out[:4]).all() and np.isfinite(out[8:]).all()
        assert m.status() == (False, False)   # the plan's last batch is clean
        # NaN in the last batch (sequence 10); then the whole call as one batch.
        ids2 = synth.make_ids(lengths, seed=3)
        ids2[10 * 40 + 3] = 777
        _o, nan2, _nb = m.embed(ids2, lengths, max_seqs=4, max_tokens=16384)
        assert nan2.tolist() == [False] * 8 + [True] * 4
        assert m.status() == (True, False)
        _o, nan3, nb3 = m.embed(ids, lengths, max_seqs=12, max_tokens=16384)
        assert nb3 == 1 and nan3.all() and m.status() == (True, False)
        m.forward(ids[:40], lengths[:1])
        assert m.status() == (False, False)
        # Several forwards on the lanes (well over 65536 tokens): the flags
        # follow the plan's batches, the vectors equal one forward per batch.
        lengths = synth.ragged_lengths(1500, seed=41, median=128.0)
        ids = synth.make_ids(lengths, seed=42)
        starts = np.concatenate([[0], np.cumsum(lengths)])
        bad_seq = 1111
        ids[starts[bad_seq] + 1] = 777
        plan = reference_plan(lengths, 512, 16384)
        log(f"embed with NaN: T={lengths.sum()} batches={len(plan)}")
        out, nan, nb = m.embed(ids, lengths, max_seqs=512, max_tokens=16384)
        assert nb == len(plan) and lengths.sum() > 3 * 65536
        want_nan = np.zeros(len(lengths), bool)
        for first, count in plan:
            if first <= bad_seq < first + count:
                want_nan[first:first + count] = True
        assert (nan == want_nan).all()
        assert np.isnan(out[bad_seq]).any() and np.isfinite(out[~want_nan]).all()
        for first, count in plan[:2] + plan[-2:]:
            want = m.forward(ids[starts[first]:starts[first + count]], lengths[first:first + count])
            np.testing.assert_array_equal(out[first:first + count], want)
    finally:
        m.close()
