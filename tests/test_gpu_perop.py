"""The per-op path: bert.go's ForwardBatch op by op through the C ABI
(longbow-fletcher_amd/perop.py: the Tensor calls the unchanged Go model makes
on this backend, internal/embeddings/model/bert.go:149-824) against the CPU
oracle at the fp32 bar (cosine >= 0.99999, max-abs <= 1e-4, reference math),
and the memory layer under it: the fl_alloc / fl_free buffer cache and the
packed weights fl_linear keeps between calls."""
import functools
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth
from longbow_fletcher_amd import perop  # noqa: E402

COS_F32, MAXABS_F32, COS_F16 = 0.99999, 1e-4, 0.999


def cosines(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1) + 1e-30)


@functools.lru_cache(maxsize=None)
def weights_for(cfg):
    return synth.make_weights(cfg)


def tiny():
    return synth.bert_tiny()


def tiny_cls():
    return synth.bert_tiny(pool=synth.POOL_CLS_TANH)


def nomic2():
    return synth.nomic(layers=2, max_pos=1024)


CASES = [
    ("bert-tiny uniform", tiny, [128] * 6),
    ("bert-tiny ragged", tiny, [128, 77, 5, 33, 1]),
    ("bert-tiny cls pooler", tiny_cls, [64] * 4),
    ("nomic 2 layers uniform", nomic2, [256] * 3),
    ("nomic 2 layers ragged", nomic2, [256, 100, 9]),
]


@pytest.mark.parametrize("name,make_cfg,lengths", CASES, ids=[c[0] for c in CASES])
def test_perop_f32_matches_oracle(ctx, fl, orc, name, make_cfg, lengths):
    cfg = make_cfg()
    lengths = np.array(lengths, np.int64)
    ids = synth.make_ids(lengths)
    print(f"per-op {name}: lengths {lengths.tolist()}", flush=True)
    m = perop.PerOpModel(ctx, cfg, weights_for(cfg), fl.F32, fl.MATH_REFERENCE)
    try:
        got = m.forward(ids, lengths)
    finally:
        m.close()
    want = orc.forward(cfg, weights_for(cfg), ids, lengths)
    c, err = cosines(got, want), float(np.abs(got - want).max())
    print(f"per-op {name}: min cos {c.min():.9f} max abs {err:.2e}", flush=True)
    assert c.min() >= COS_F32 and err <= MAXABS_F32


def test_perop_f16_nomic_matches_oracle_and_model(ctx, fl, orc):
    cfg = nomic2()
    lengths = np.array([512, 512, 512, 512], np.int64)
    ids = synth.make_ids(lengths)
    m = perop.PerOpModel(ctx, cfg, weights_for(cfg), fl.F16, fl.MATH_EXACT)
    try:
        got = m.forward(ids, lengths)
        again = m.forward(ids, lengths)  # packed weights now come from the cache
    finally:
        m.close()
    np.testing.assert_array_equal(got, again)
    want = orc.forward(cfg, weights_for(cfg), ids, lengths)
    assert cosines(got, want).min() >= COS_F16
    model = fl.Model(ctx, cfg, dtype=fl.F16, math=fl.MATH_EXACT)
    try:
        model.load(weights_for(cfg))
        fused = model.forward(ids, lengths)
    finally:
        model.close()
    c = cosines(got, fused)
    print(f"per-op vs model-level fp16: min cos {c.min():.7f}", flush=True)
    assert c.min() >= 0.9999


def test_pool_reuses_freed_blocks_zeroed(ctx, fl):
    a = ctx.tensor(np.full((1000, 256), 3.0, np.float32), fl.F32)
    a.free()
    s0 = ctx.pool_stats()
    b = ctx.empty((1000, 256), fl.F32)
    s1 = ctx.pool_stats()
    try:
        assert s1["hits"] == s0["hits"] + 1 and s1["misses"] == s0["misses"]
        assert s1["live_buffers"] == s0["live_buffers"] + 1
        # GetTensor hands out zeros (device_test.go:98-112), reused blocks too.
        assert not np.any(b.numpy())
    finally:
        b.free()


def test_pool_trim_returns_cached_bytes(ctx, fl):
    t = ctx.empty((4096, 1024), fl.F32)
    t.free()
    held = ctx.vram_usage()[0]
    cached = ctx.pool_stats()["cached_bytes"]
    assert cached >= 4096 * 1024 * 4
    ctx.pool_trim()
    assert ctx.vram_usage()[0] == held - cached
    assert ctx.pool_stats()["cached_bytes"] == 0


def _upload(fl, ctx, t, data):
    a = np.ascontiguousarray(data, np.float32)
    fl.check(fl.lib().fl_upload_f32(ctx.h, t.ptr, t.dtype, a.ctypes.data, a.size,
                                    fl.ROUND_NEAREST))


@pytest.mark.parametrize("dtype_name", ["F16", "F32"])
def test_linear_weight_cache_follows_writes(ctx, fl, dtype_name):
    """A weight's packed copy is reused while the weight is unchanged and
    rebuilt after any write through the ABI; freeing the weight releases it."""
    dtype = getattr(fl, dtype_name)
    math_mode = fl.MATH_EXACT if dtype != fl.F32 else fl.MATH_REFERENCE
    rng = np.random.default_rng(3)
    x = ctx.tensor(rng.standard_normal((300, 256)).astype(np.float32), dtype)
    # Away from fp16's subnormal range, where rounding 2x and doubling the
    # rounded x can differ.
    def weights():
        w = rng.standard_normal((256, 512)) * 0.05
        return (np.sign(w) * np.maximum(np.abs(w), 1e-3)).astype(np.float32)

    w1, w2 = weights(), weights()
    b1 = rng.standard_normal((1, 512)).astype(np.float32)
    b2 = rng.standard_normal((1, 512)).astype(np.float32)
    W = ctx.tensor(w1, dtype)
    b = ctx.tensor(b1, dtype)

    def lin(w, bias):
        y = ctx.linear(x, w, bias, math=math_mode)
        out = y.numpy()
        y.free()
        return out

    def fresh(wdata, bdata):
        tw, tb = ctx.tensor(wdata, dtype), ctx.tensor(bdata, dtype)
        try:
            return lin(tw, tb)
        finally:
            tw.free()
            tb.free()

    try:
        p0 = ctx.pool_stats()["packed_bytes"]
        y1 = lin(W, b)
        p1 = ctx.pool_stats()["packed_bytes"]
        assert p1 > p0  # the bias at least is kept packed (fp32, packed order)
        np.testing.assert_array_equal(lin(W, b), y1)  # from the cache
        np.testing.assert_array_equal(y1, fresh(w1, b1))
        _upload(fl, ctx, W, w2)  # Tensor.CopyFromFloat32
        np.testing.assert_array_equal(lin(W, b), fresh(w2, b1))
        ctx.scale(W, 2.0)  # Tensor.Scale in place
        np.testing.assert_array_equal(lin(W, b), fresh(2.0 * w2, b1))
        _upload(fl, ctx, b, b2)  # the bias is tracked the same way
        np.testing.assert_array_equal(lin(W, b), fresh(2.0 * w2, b2))
        W.free()
        b.free()
        W = b = None
        assert ctx.pool_stats()["packed_bytes"] == p0
    finally:
        for t in (x, b, W):
            if t is not None:
                t.free()
