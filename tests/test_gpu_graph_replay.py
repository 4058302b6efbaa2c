"""Captured forwards (model.cpp run_graphed): synchronous forwards of up to
4096 tokens replay a HIP graph of their kernels, captured the first time a
lengths vector is seen.  Every replay must give the bits of the same forward
run eagerly (fl_model_forward_device runs the kernels directly), also with
other work and synchronisations between replays, new ids in the same shape,
and after a larger forward has moved the lane's buffers (a new capture)."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth


def eager(fl, ctx, m, ids, lengths, H):
    d_ids = ctx.int32(np.asarray(ids, np.int32))
    d_out = ctx.empty((len(lengths), H), fl.F32)
    try:
        m.forward_device(d_ids, lengths, d_out)
        return d_out.numpy()
    finally:
        d_ids.free()
        d_out.free()


@pytest.mark.parametrize("dtype_name,make_cfg", [("F16", lambda: synth.nomic(layers=2)),
                                                 ("F32", lambda: synth.bert_tiny())])
def test_graph_replays_match_eager(fl, ctx, dtype_name, make_cfg):
    cfg = make_cfg()
    dtype = getattr(fl, dtype_name)
    math_mode = fl.MATH_EXACT if dtype != fl.F32 else fl.MATH_REFERENCE
    m = fl.Model(ctx, cfg, dtype=dtype, math=math_mode)
    rng = np.random.default_rng(5)
    try:
        m.load(synth.make_weights(cfg))
        for lengths in (np.array([16], np.int64), np.array([128, 7, 300], np.int64)):
            print(f"graph replay {cfg.name} {dtype_name} lengths {lengths.tolist()}", flush=True)
            for rep in range(4):
                ids = rng.integers(1000, 30000, int(lengths.sum())).astype(np.int64)
                got = m.forward(ids, lengths)  # first: capture, then replays
                # Eager work of the program between replays.
                x = ctx.tensor(rng.standard_normal((64, 256)).astype(np.float32), fl.F16)
                ctx.scale(x, 2.0)
                ctx.synchronize()
                x.free()
                want = eager(fl, ctx, m, ids, lengths, cfg.hidden)
                np.testing.assert_array_equal(got, want)
                np.testing.assert_array_equal(m.forward(ids, lengths), want)
        # A forward past the graph limit (not captured) grows the lane's
        # buffers; the small shape is captured again at the new addresses.
        big = np.array([3000, 2000], np.int64)
        ids_big = rng.integers(1000, 30000, int(big.sum())).astype(np.int64)
        np.testing.assert_array_equal(m.forward(ids_big, big),
                                      eager(fl, ctx, m, ids_big, big, cfg.hidden))
        lengths = np.array([16], np.int64)
        ids = rng.integers(1000, 30000, 16).astype(np.int64)
        np.testing.assert_array_equal(m.forward(ids, lengths),
                                      eager(fl, ctx, m, ids, lengths, cfg.hidden))
    finally:
        m.close()
