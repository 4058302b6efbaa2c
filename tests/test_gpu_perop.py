"""The per-op path: bert.go's ForwardBatch op by op through the C ABI
(longbow-fletcher_amd/perop.py replays the Tensor calls the unchanged Go model
makes, internal/embeddings/model/bert.go:149-824, through device.py, the
mirror of the Go binding) against the CPU oracle, and the memory layer under
it: the fl_alloc / fl_free buffer cache, the packed weights and converted
activations fl_linear keeps between calls, views, operand extent checks.

Bars: fp32 with reference math cos >= 0.99999 and max-abs <= 1e-4; fp16
cos >= 0.999 against the fp32 oracle."""
import functools
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth
from longbow_fletcher_amd import device, perop  # noqa: E402

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


@pytest.fixture(scope="module")
def be32():
    b = device.RocmBackend(0, device.Float32)
    yield b
    b.close()


def backend_for(cfg, dtype):
    return device.RocmBackend(0, dtype, rope_base=cfg.rope_base)


# (name, config, lengths, mode): uniform batches take bert.go's own path in
# either mode; mixed lengths compare the "intended" mode with the oracle's
# forward (per-sequence multi-head attention, the model-level semantics).
CASES = [
    ("bert-tiny uniform", tiny, [128] * 6, "literal"),
    ("bert-tiny ragged intended", tiny, [128, 77, 5, 33, 1], "intended"),
    ("bert-tiny cls pooler", tiny_cls, [64] * 4, "literal"),
    ("nomic 2 layers uniform", nomic2, [256] * 3, "literal"),
    ("nomic 2 layers ragged intended", nomic2, [256, 100, 9], "intended"),
]


@pytest.mark.parametrize("name,make_cfg,lengths,mode", CASES, ids=[c[0] for c in CASES])
def test_perop_f32_matches_oracle(fl, orc, name, make_cfg, lengths, mode):
    cfg = make_cfg()
    lengths = np.array(lengths, np.int64)
    ids = synth.make_ids(lengths)
    print(f"per-op {name}: lengths {lengths.tolist()}", flush=True)
    b = backend_for(cfg, device.Float32)
    m = perop.PerOpModel(b, cfg, weights_for(cfg), mode=mode)
    try:
        got = m.forward(ids, lengths)
    finally:
        m.close()
        b.close()
    want = orc.forward(cfg, weights_for(cfg), ids, lengths)
    c, err = cosines(got, want), float(np.abs(got - want).max())
    print(f"per-op {name}: min cos {c.min():.9f} max abs {err:.2e}", flush=True)
    assert c.min() >= COS_F32 and err <= MAXABS_F32


def literal_oracle(orc, cfg, w, ids, lengths, attn_out=None):
    """bert.go's ForwardBatch for an fp32 absolute-position model, composed
    from the oracle's Tensor ops in bert.go's order, mixed-length branch
    (:653-720) included: per sequence, Q and K scaled by
    float32(sqrt(float64(scale))), scores = Q K^T over all H columns,
    SoftmaxFast, times V.  Pools as cfg.pool (mean + L2 in float64)."""
    H, heads = cfg.hidden, cfg.heads
    hd = H // heads
    T = int(lengths.sum())
    zero = np.zeros((1, H), np.float32)
    one = np.ones((1, H), np.float32)
    g = lambda n, d: w.get(n, d)  # noqa: E731
    h = orc.gather(w["word_emb"], ids)
    pos = np.concatenate([np.minimum(np.arange(L), cfg.max_pos - 1) for L in lengths])
    h = orc.add(h, orc.gather(w["pos_emb"], pos))
    h = orc.add(h, orc.gather(w["type_emb"], np.zeros(T, np.int64)))
    h = orc.layernorm(h, g("emb_ln_g", one), g("emb_ln_b", zero), 1e-7)
    scale = np.float32(1.0) / np.float32(np.sqrt(np.float64(hd)))
    ss = np.float32(np.sqrt(np.float64(scale)))
    for l in range(cfg.layers):
        q = orc.linear(h, w[f"q_w.{l}"], w[f"q_b.{l}"])
        k = orc.linear(h, w[f"k_w.{l}"], w[f"k_b.{l}"])
        v = orc.linear(h, w[f"v_w.{l}"], w[f"v_b.{l}"])
        out = np.zeros((T, H), np.float32)
        off = 0
        for L in (int(x) for x in lengths):
            qs = orc.scale(q[off:off + L], ss)
            ks = orc.scale(k[off:off + L], ss)
            scores = orc.softmax_rows(orc.mul(qs, ks, trans_b=True))
            out[off:off + L] = orc.mul(scores, v[off:off + L])
            off += L
        if attn_out is not None:
            attn_out.append(out)
        o = orc.linear(out, w[f"o_w.{l}"], w[f"o_b.{l}"])
        h = orc.add_layernorm(h, o, g(f"attn_ln_g.{l}", one), g(f"attn_ln_b.{l}", zero), 1e-7)
        inter = orc.linear_activation(h, w[f"inter_w.{l}"], w[f"inter_b.{l}"], cfg.activation)
        o2 = orc.linear(inter, w[f"out_w.{l}"], w[f"out_b.{l}"])
        h = orc.add_layernorm(h, o2, g(f"out_ln_g.{l}", one), g(f"out_ln_b.{l}", zero), 1e-7)
    starts = np.concatenate([[0], np.cumsum(lengths)])
    p = np.stack([h[starts[i]:starts[i + 1]].astype(np.float64).mean(0)
                  for i in range(len(lengths))])
    if cfg.pool == synth.POOL_MEAN_L2:
        p = p / np.maximum(np.linalg.norm(p, axis=1, keepdims=True), 1e-12)
    return p


def test_perop_literal_mixed_lengths_f32(fl, orc):
    """bert.go as written on a mixed-length batch (bert-tiny, fp32): the
    Slice views of Q, K, V are scaled in place and the attention result is
    written through a Slice view of the output, so every attention output row
    is non-zero, and the pooled vectors match the same op sequence on the
    oracle."""
    cfg = tiny()
    lengths = np.array([128, 77, 5, 33, 1, 64], np.int64)
    ids = synth.make_ids(lengths)
    w = weights_for(cfg)
    seen = []

    def probe(layer, t):
        n, c = t.Dims()
        seen.append(t.ToHost().reshape(n, c))

    b = backend_for(cfg, device.Float32)
    m = perop.PerOpModel(b, cfg, w, mode="literal", on_attention=probe)
    try:
        got = m.forward(ids, lengths)
    finally:
        m.close()
        b.close()
    want_attn = []
    want = literal_oracle(orc, cfg, w, ids, lengths, want_attn)
    assert len(seen) == cfg.layers
    for li, (a, wa) in enumerate(zip(seen, want_attn)):
        zero_rows = int((np.abs(a).max(1) == 0).sum())
        err = float(np.abs(a - wa).max())
        print(f"layer {li}: attention zero rows {zero_rows}, max abs vs oracle {err:.2e}",
              flush=True)
        assert zero_rows == 0
        assert err <= MAXABS_F32
    c, err = cosines(got, want), float(np.abs(got - want).max())
    print(f"literal mixed lengths: min cos {c.min():.9f} max abs {err:.2e}", flush=True)
    assert c.min() >= COS_F32 and err <= MAXABS_F32


def test_perop_f16_nomic_literal_matches_oracle_and_model(fl, orc):
    """bert.go on an fp16 backend, uniform 2-layer Nomic batch: fp16 weights,
    the fp32 master stream of bert.go:253-258 (fp32 hidden state into fp16
    Linear, fp16 branches added to it by AddLayerNorm)."""
    cfg = nomic2()
    lengths = np.array([512, 512, 512, 512], np.int64)
    ids = synth.make_ids(lengths)
    b = backend_for(cfg, device.Float16)
    m = perop.PerOpModel(b, cfg, weights_for(cfg))
    try:
        got = m.forward(ids, lengths)
        again = m.forward(ids, lengths)  # packed weights now come from the cache
        assert b.GetVRAMUsage()[0] > 0
    finally:
        m.close()
        b.close()
    np.testing.assert_array_equal(got, again)
    want = orc.forward(cfg, weights_for(cfg), ids, lengths)
    c = cosines(got, want)
    print(f"per-op fp16 literal vs oracle: min cos {c.min():.7f}", flush=True)
    assert c.min() >= COS_F16
    ctx = fl.Context(0)
    model = fl.Model(ctx, cfg, dtype=fl.F16, math=fl.MATH_EXACT)
    try:
        model.load(weights_for(cfg))
        fused = model.forward(ids, lengths)
    finally:
        model.close()
        ctx.close()
    c = cosines(got, fused)
    print(f"per-op vs model-level fp16: min cos {c.min():.7f}", flush=True)
    assert c.min() >= 0.9999


def test_linear_rejects_short_weight_buffer(fl, ctx):
    """An fp16 weight passed as fp32 would be read past its end: fl_linear
    returns FL_ERR_INVALID on the host and enqueues nothing."""
    rows, k, n = 64, 256, 256
    x = ctx.tensor(np.ones((rows, k), np.float32), fl.F32)
    w16 = ctx.tensor(np.full((k, n), 0.5, np.float32), fl.F16)
    out = ctx.tensor(np.full((rows, n), 7.0, np.float32), fl.F32)
    try:
        ctx.synchronize()
        before = ctx.pool_stats()
        rc = fl.lib().fl_linear(ctx.h, fl.F32, x.ptr, rows, k, fl.F32, w16.ptr, fl.W_IN_OUT, n,
                                None, fl.ACT_IDENTITY, fl.MATH_REFERENCE, out.ptr)
        msg = fl.lib().fl_last_error().decode()
        print(f"rejected: rc {rc}: {msg}", flush=True)
        assert rc == fl.ERR_INVALID and "W" in msg and "past the end" in msg
        assert ctx.pool_stats() == before  # nothing packed, nothing allocated
        np.testing.assert_array_equal(out.numpy(), 7.0)  # nothing ran
        # The same weight with its real type runs.
        y = ctx.linear(x, w16)
        assert y.dtype == fl.F16
        np.testing.assert_allclose(y.numpy(), 0.5 * k, rtol=1e-3)
        y.free()
        # Every per-op operand is checked: a short bias, x, output.
        for args in ((fl.F32, x.ptr, rows + 1, k, fl.F16, w16.ptr),
                     (fl.F16, x.ptr, rows * 2 + 1, k, fl.F16, w16.ptr)):
            rc = fl.lib().fl_linear(ctx.h, args[0], args[1], args[2], args[3], args[4], args[5],
                                    fl.W_IN_OUT, n, None, 0, fl.MATH_EXACT, out.ptr)
            assert rc == fl.ERR_INVALID
        rc = fl.lib().fl_add(ctx.h, fl.F32, out.ptr, fl.F16, w16.ptr, 2 * rows * n)
        assert rc == fl.ERR_INVALID
        np.testing.assert_array_equal(out.numpy(), 7.0)
    finally:
        for t in (x, w16, out):
            t.free()


def test_views_mixed_types_and_converted_copy(fl, orc):
    """Slice of whole rows is a view: writes through it (Scale, Copy) land in
    the parent.  Add / AddLayerNorm convert the other operand to the
    receiver's type.  A 16-bit Linear reading an fp32 tensor reuses one
    converted copy, which a LayerNorm of that tensor rewrites in its pass."""
    b = device.RocmBackend(0, device.Float16)
    rng = np.random.default_rng(11)
    try:
        H = 768
        x = rng.standard_normal((300, H)).astype(np.float32)
        h = b.NewTensorWithType(300, H, device.Float32, x)
        v = h.Slice(100, 200, 0, H)
        v.Scale(2.0)
        y = h.ToHost().reshape(300, H)
        np.testing.assert_array_equal(y[100:200], 2.0 * x[100:200])
        np.testing.assert_array_equal(y[:100], x[:100])
        np.testing.assert_array_equal(y[200:], x[200:])
        # Copy through a view of another tensor's rows.
        src = b.NewTensorWithType(100, H, device.Float32, x[:100])
        h.Slice(200, 300, 0, H).Copy(src)
        np.testing.assert_array_equal(h.ToHost().reshape(300, H)[200:], x[:100])
        # Column slices are copies (fl_slice).
        cs = h.Slice(0, 300, 64, 128)
        np.testing.assert_array_equal(cs.ToHost().reshape(300, 64),
                                      h.ToHost().reshape(300, H)[:, 64:128])
        # Add: fp32 receiver, fp16 other (converted on load).
        r16 = b.NewTensor(300, H, rng.standard_normal((300, H)).astype(np.float32))
        hv = h.ToHost().reshape(300, H)
        h.Add(r16)
        want = orc.add(hv, r16.ToHost().reshape(300, H))
        np.testing.assert_array_equal(h.ToHost().reshape(300, H), want)
        # AddLayerNorm, fp32 receiver + fp16 branch, against the oracle.
        g = b.NewTensorWithType(1, H, device.Float32, np.ones(H, np.float32))
        z = b.NewTensorWithType(1, H, device.Float32, np.zeros(H, np.float32))
        hv = h.ToHost().reshape(300, H)
        h.AddLayerNorm(r16, g, z, 1e-7)
        want = orc.add_layernorm(hv, r16.ToHost().reshape(300, H), np.ones(H), np.zeros(H),
                                 1e-7)
        np.testing.assert_allclose(h.ToHost().reshape(300, H), want, atol=2e-5, rtol=1e-5)
        # fp16 Linear of the fp32 h: one converted copy, shared by two calls.
        W = b.NewTensor(H, H, (rng.standard_normal((H, H)) * 0.02).astype(np.float32))
        def packed_bytes():
            st = (fl.C.c_int64 * 6)()
            fl.check(fl.lib().fl_pool_stats(b.ctx, st))
            return st[4]

        p0 = packed_bytes()
        y1 = W.Linear(h, W, None)
        p1 = packed_bytes()
        y2 = W.Linear(h, W, None)
        assert packed_bytes() == p1 > p0
        assert y1.DataType() == device.Float16
        np.testing.assert_array_equal(y1.ToHost(), y2.ToHost())

        def fresh():
            h16 = h.Cast(device.Float16)
            y = W.Linear(h16, W, None).ToHost()
            b.PutTensor(h16)
            return y

        np.testing.assert_array_equal(y1.ToHost(), fresh())
        # The LayerNorm rewrites h and its copy: the next Linear reads the
        # new values, with the copy made by the LayerNorm's own store.
        h.AddLayerNorm(r16, g, z, 1e-7)
        y3 = W.Linear(h, W, None)
        assert packed_bytes() == p1
        np.testing.assert_array_equal(y3.ToHost(), fresh())
        # Scale through a view also invalidates the copy.
        h.Slice(0, 10, 0, H).Scale(3.0)
        np.testing.assert_array_equal(W.Linear(h, W, None).ToHost(), fresh())
    finally:
        b.close()


def test_tensor_method_set(fl):
    """At, Set, ExtractTo, ExtractToFlat, ExtractBytes, T and HasNaN of the
    binding (device.go:5-117), fp32 and fp16."""
    b = device.RocmBackend(0, device.Float16)
    try:
        a = np.arange(12, dtype=np.float32).reshape(3, 4) / 4
        for dt in (device.Float32, device.Float16):
            t = b.NewTensorWithType(3, 4, dt, a)
            assert t.At(2, 1) == a[2, 1]
            assert t.T().At(1, 2) == a[2, 1] and t.T().Dims() == (4, 3)
            t.Set(1, 3, -5.5)
            assert t.At(1, 3) == -5.5
            rows = [None] * 5
            t.ExtractTo(rows, 1)
            assert rows[0] is None and np.array_equal(rows[2], [1.0, 1.25, 1.5, -5.5])
            flat = np.zeros(14, np.float32)
            t.ExtractToFlat(flat, 2)
            assert flat[2 + 7] == -5.5 and flat[2] == 0.0
            raw = t.ExtractBytes()
            want = a.copy()
            want[1, 3] = -5.5
            npdt = np.float32 if dt == device.Float32 else np.float16
            assert raw == want.astype(npdt).tobytes()
            np.testing.assert_array_equal(t.T().ToHost(), want.T.ravel())
            assert t.HasNaN() == (False, None)
            t.Set(0, 0, float("nan"))
            assert t.HasNaN()[0]
            b.PutTensor(t)
        # GetTensor hands out zeros; a view is never freed by PutTensor.
        z = b.GetTensor(8, 8)
        v = z.Slice(2, 4, 0, 8)
        b.PutTensor(v)
        assert not np.any(z.ToHost())
        b.PutTensor(z)
    finally:
        b.close()


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
