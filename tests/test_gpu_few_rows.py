"""GPU checks of the few-row GEMM path: a forward of a few hundred tokens runs
some or all of its 16-bit projections on the few-row kernel (chosen per GEMM
from the rows, width and depth), one of more than 4096 tokens all of them on
the persistent four-wave kernel.  Both multiply in the same MFMA and K order
and share the epilogue math, so a sequence's last hidden states and vector
must be the
same bits whether it runs alone or inside a large batch (the property the
embedding batching relies on: runInferenceOnDevice,
internal/embeddings/embeddings.go:704-775, splits requests into batches
freely).  Each family covers other epilogues: Nomic (RoPE with the query
scale, SwiGLU with the tiled output, no bias), BERT-base (bias, GELU, query
scale in the plain epilogue), MiniLM (padded 384- and 1152-wide
projections)."""
import sys
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth

LENGTHS = [1, 7, 16, 100, 255, 256, 300, 512]
FILL = [512] * 8   # takes the batch past 4096 tokens: four-wave kernel only


def log(msg):
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)


@pytest.mark.parametrize("family,dtype", [("nomic", "f16"), ("bert_base", "f16"),
                                          ("minilm", "f16"), ("nomic", "bf16")])
def test_alone_equals_in_batch(fl, ctx, family, dtype):
    cfg = getattr(synth, family)(layers=2)
    w = synth.make_weights(cfg)
    m = fl.Model(ctx, cfg, dtype=fl.F16 if dtype == "f16" else fl.BF16)
    try:
        m.load(w)
        lengths = np.array(LENGTHS + FILL, np.int64)
        ids = synth.make_ids(lengths, seed=51)
        starts = np.concatenate([[0], np.cumsum(lengths)])
        log(f"{family}: batch of {len(lengths)} sequences, T={lengths.sum()}")
        big = m.forward(ids, lengths)
        hid = m.last_hidden(int(lengths.sum()))
        for i, n in enumerate(LENGTHS):
            log(f"{family}: sequence {i} alone, {n} tokens")
            alone = m.forward(ids[starts[i]:starts[i + 1]], lengths[i:i + 1])
            np.testing.assert_array_equal(alone[0], big[i])
            np.testing.assert_array_equal(m.last_hidden(n), hid[starts[i]:starts[i + 1]])
        # Several short sequences together (24 tokens), and the eight of
        # LENGTHS (1447 tokens: FFN-down and O on the few-row kernel, FFN-up
        # on the four-wave one), against the same batch.
        for k in (4, len(LENGTHS)):
            part = m.forward(ids[:starts[k]], lengths[:k])
            np.testing.assert_array_equal(part, big[:k])
    finally:
        m.close()
