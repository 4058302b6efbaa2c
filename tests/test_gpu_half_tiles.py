"""GPU checks of the half tiles of the four-wave GEMM (gemm.hip, launch_w4):
a STORE GEMM with K <= 1024 whose 256x256 tiles leave a partial last round
of at most half the CUs runs that round as 256x128 half tiles, two per tile,
each the last tile of its workgroup.  Both multiply in the same
MFMA and K order and share the epilogue math, so every output row must have
the same bits whichever kernel computed it.  Output rows depend only on
their own input row, so a GEMM over the first rows of a larger input is
compared with the rows of the larger GEMM.

Tile counts below assume MI355X's 256 CUs (on a device with another count
the split lands elsewhere, and the equalities still hold)."""
import sys
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth


def log(msg):
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)


@pytest.mark.parametrize("dtype_name", ["F16", "BF16"])
@pytest.mark.parametrize("n", [768, 2304])
def test_split_rounds_match_whole_rounds(fl, ctx, dtype_name, n):
    dtype = getattr(fl, dtype_name)
    rng = np.random.default_rng(11)
    k = 768
    # 256 row blocks: 3 (or 9) column tiles each, whole rounds only.
    big = 256 * 256
    w = (rng.standard_normal((k, n)) * 0.05).astype(np.float32)
    b = rng.standard_normal((1, n)).astype(np.float32)
    x = rng.standard_normal((big, k)).astype(np.float32)
    X, W, B = ctx.tensor(x, dtype), ctx.tensor(w, dtype), ctx.tensor(b, dtype)
    ts = [X, W, B]
    try:
        log(f"{dtype_name} N={n}: {big} rows (whole rounds)")
        ref = ctx.linear(X, W, B)
        ts.append(ref)
        want = ref.numpy().reshape(big, n)
        # 128 row blocks (N=768: 384 tiles = one round + 128 tiles as half
        # tiles; N=2304: 1152 = four rounds + 128), 8 (half tiles only),
        # 8 with the last block ragged, and without a bias.
        for rows in (128 * 256, 8 * 256, 7 * 256 + 200):
            log(f"{dtype_name} N={n}: first {rows} rows")
            out = ctx.linear(X.rows_view(0, rows), W, B)
            np.testing.assert_array_equal(out.numpy().reshape(rows, n), want[:rows])
            out.free()
        nob = ctx.linear(X, W)
        part = ctx.linear(X.rows_view(0, 7 * 256 + 200), W)
        np.testing.assert_array_equal(part.numpy().reshape(-1, n),
                                      nob.numpy().reshape(big, n)[:7 * 256 + 200])
        nob.free()
        part.free()
    finally:
        for t in ts:
            t.free()


def test_bert_base_batch_equals_alone(fl, ctx):
    """BERT-base at the bench's batch (256 x 128 tokens): QKV (1152 tiles,
    with the query scale) and O (384 tiles) end in a round of half tiles; the
    same sequences alone or 16 at a time take the few-row kernel or half
    tiles only."""
    cfg = synth.bert_base(layers=2)
    w = synth.make_weights(cfg)
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    try:
        m.load(w)
        lengths = np.full(256, 128, np.int64)
        ids = synth.make_ids(lengths, seed=53)
        log("bert_base: 256 x 128 tokens")
        big = m.forward(ids, lengths)
        hid = m.last_hidden(int(lengths.sum()))
        for i in (0, 97, 255):
            log(f"bert_base: sequence {i} alone")
            alone = m.forward(ids[i * 128:(i + 1) * 128], lengths[i:i + 1])
            np.testing.assert_array_equal(alone[0], big[i])
            np.testing.assert_array_equal(m.last_hidden(128), hid[i * 128:(i + 1) * 128])
        log("bert_base: sequences 16-31 together")
        part = m.forward(ids[16 * 128:32 * 128], lengths[16:32])
        np.testing.assert_array_equal(part, big[16:32])
    finally:
        m.close()
