"""Device memory pressure: the library's allocations give cached memory back
before they fail.

* Freed fl_alloc blocks and packed weights (the per-op path's caches) fill
  the device, then a model is created and runs: its allocations trim the
  cache and drop the packed copies instead of failing.
* fl_model_embed on a device that cannot hold its lanes' activation buffers
  falls back to one forward per batch on the context stream, with the same
  output bits.
* fl_model_last_hidden after fl_model_embed returns the plan's last forward.
"""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth
GIB = 1 << 30
MIB = 1 << 20


def mem_free():
    """hipMemGetInfo's free bytes of the current device (the library has made
    device 0 current on this thread)."""
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def fill(fl, ctx, leave=8 * MIB, sizes=(4 * GIB, 256 * MIB, 16 * MIB)):
    """Live fl_alloc_uninit blocks until less than `leave` + the smallest
    size stays free.  No allocation is made that would not fit, so none
    fails (a failing one would make the library drop its packed copies)."""
    blocks = []
    for sz in sizes:
        while mem_free() - sz >= leave:
            blocks.append(ctx.result((sz // 2,), fl.F16))
    return blocks


def test_model_created_after_caches_fill_device(fl, orc):
    ctx = fl.Context(0)
    blocks = []
    try:
        rng = np.random.default_rng(1)
        x = ctx.tensor(rng.standard_normal((256, 2048)).astype(np.float32), fl.F16)
        ws = [ctx.tensor(rng.standard_normal((2048, 8192)).astype(np.float32) * 0.02, fl.F16)
              for _ in range(3)]
        for w in ws:
            ctx.linear(x, w, math=fl.MATH_EXACT).free()
        ctx.synchronize()
        packed = ctx.pool_stats()["packed_bytes"]
        assert packed >= 3 * 2048 * 8192 * 2
        blocks = fill(fl, ctx)
        print(f"filled: {len(blocks)} blocks, {mem_free() / MIB:.0f} MiB free", flush=True)
        assert mem_free() < 64 * MIB
        assert ctx.pool_stats()["packed_bytes"] == packed
        for b in blocks:
            b.free()
        blocks = []
        st = ctx.pool_stats()
        print(f"cached {st['cached_bytes'] / GIB:.1f} GiB, packed {packed / MIB:.0f} MiB, "
              f"free {mem_free() / MIB:.0f} MiB", flush=True)
        assert mem_free() < 64 * MIB
        # A model now: its allocations find the device full and take the
        # cached blocks and packed copies back.
        cfg = synth.nomic(layers=2, max_pos=1024)
        w = synth.make_weights(cfg)
        lengths = np.array([300, 512, 77], np.int64)
        ids = synth.make_ids(lengths)
        m = fl.Model(ctx, cfg, dtype=fl.F16)
        try:
            m.load(w)
            got = m.forward(ids, lengths)
        finally:
            m.close()
        want = orc.forward(cfg, w, ids, lengths)
        cos = (got * want).sum(1) / np.linalg.norm(got, axis=1) / np.linalg.norm(want, axis=1)
        print(f"model after eviction: min cos {cos.min():.7f}, packed "
              f"{ctx.pool_stats()['packed_bytes']} bytes", flush=True)
        assert cos.min() >= 0.999
        assert ctx.pool_stats()["packed_bytes"] < packed
        # The per-op path still works (packs again).
        y = ctx.linear(x, ws[0], math=fl.MATH_EXACT)
        assert np.isfinite(y.numpy()).all()
        y.free()
        for t in ws + [x]:
            t.free()
    finally:
        for b in blocks:
            b.free()
        ctx.pool_trim()
        ctx.close()


def test_embed_falls_back_when_lanes_do_not_fit(fl):
    """Two 65536-token forwards on two lanes need ~2.2 GB of activations
    (Nomic fp16); with ~600 MiB free, fl_model_embed runs the plan's eight
    16384-token batches one by one on lane 0 instead."""
    cfg = synth.nomic(layers=2)
    w = synth.make_weights(cfg)
    lengths = np.full(256, 512, np.int64)
    ids = synth.make_ids(lengths)
    ctx = fl.Context(0)
    blocks = []
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    try:
        m.load(w)
        m.forward(ids[:1024], lengths[:2])  # weights packed, tables made
        blocks = fill(fl, ctx, leave=600 * MIB, sizes=(4 * GIB, 256 * MIB, 16 * MIB))
        print(f"{mem_free() / MIB:.0f} MiB free", flush=True)
        out, nan, nb = m.embed(ids, lengths, 512, 16384)
        assert nb == 8 and not nan.any()
        for b in blocks:
            b.free()
        blocks = []
        ctx.pool_trim()
        grouped, _, _ = m.embed(ids, lengths, 512, 16384)
        np.testing.assert_array_equal(out, grouped)
        first = m.forward(ids[:16384], lengths[:32])
        np.testing.assert_array_equal(out[:32], first)
    finally:
        for b in blocks:
            b.free()
        m.close()
        ctx.pool_trim()
        ctx.close()


def test_last_hidden_after_embed_is_last_forward(fl, ctx):
    cfg = synth.nomic(layers=2)
    w = synth.make_weights(cfg)
    lengths = np.full(160, 512, np.int64)  # forwards of 65536 and 16384 tokens
    ids = synth.make_ids(lengths)
    m = fl.Model(ctx, cfg, dtype=fl.F16)
    try:
        m.load(w)
        m.embed(ids, lengths, 512, 16384)
        tail = m.last_hidden(32 * 512)
        m.forward(ids[128 * 512:], lengths[128:])
        np.testing.assert_array_equal(tail, m.last_hidden(32 * 512))
    finally:
        m.close()
